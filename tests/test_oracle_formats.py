"""Pins the oracle's number formats (CPU).

* e4m3fn encode: the C restatement (written from the OCP format definition)
  against torch's own float -> float8_e4m3fn cast on every bf16 value, on
  350k random float32 values and on the known answers of the format
  (max 448, smallest subnormal 2^-9, ties to even, overflow -> NaN).
* e4m3fn decode: all 256 codes against torch.
* bf16 rounding: every float32 in a random sample plus the tie cases against
  torch's cast.
* The reference's quantisation conventions (oracle/fp8.py: multiply by a
  reciprocal in the activation dtype, or divide by the dequant scale in
  fp32, clamp to +-448) against the C restatement.
"""
import numpy as np
import pytest
import torch

from oracle import c_oracle as C
from oracle import fp8 as F


def _torch_e4m3(x_f32: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x_f32).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _same_bytes_nan_aware(a: np.ndarray, b: np.ndarray):
    # NaN codes: 0x7F / 0xFF; torch keeps the input's sign on NaN
    assert a.shape == b.shape
    bad = np.nonzero(a != b)[0]
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:5]}: {a[bad[:5]]} vs {b[bad[:5]]}"


def test_e4m3fn_known_answers():
    kat = [
        (0.0, 0x00), (-0.0, 0x80), (1.0, 0x38), (-1.0, 0xB8), (448.0, 0x7E), (-448.0, 0xFE),
        (2.0 ** -9, 0x01), (2.0 ** -6, 0x08), (7 * 2.0 ** -9, 0x07), (0.5, 0x30), (1.125, 0x39),
        # ties to even: 1.0625 is halfway between 1.0 (0x38) and 1.125 (0x39)
        (1.0625, 0x38), (1.1875, 0x3A),
        # 464 is halfway between 448 and the NaN code: even mantissa -> 448
        (464.0, 0x7E),
        # half the smallest subnormal rounds to zero (tie to even), just above to 2^-9
        (2.0 ** -10, 0x00), (2.0 ** -10 * 1.0001, 0x01),
    ]
    xs = np.array([k for k, _ in kat], dtype=np.float32)
    got = C.e4m3fn_from_f32(xs)
    exp = np.array([v for _, v in kat], dtype=np.uint8)
    np.testing.assert_array_equal(got, exp)
    np.testing.assert_array_equal(_torch_e4m3(xs), exp)
    for v in (465.0, 480.0, 1e6, float("inf"), float("nan")):
        assert C.e4m3fn_from_f32(np.array([v], np.float32))[0] & 0x7F == 0x7F


def test_e4m3fn_encode_all_bf16_values():
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    xs = bits.view(np.float32)
    _same_bytes_nan_aware(C.e4m3fn_from_f32(xs), _torch_e4m3(xs))


def test_e4m3fn_encode_random_f32():
    rng = np.random.default_rng(5)
    xs = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * 100,
        rng.uniform(-2 ** -5, 2 ** -5, 100_000).astype(np.float32),   # subnormal range
        rng.uniform(400, 520, 50_000).astype(np.float32),              # overflow edge
    ])
    _same_bytes_nan_aware(C.e4m3fn_from_f32(xs), _torch_e4m3(xs))


def test_e4m3fn_decode_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = C.f32_from_e4m3fn(codes)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok], ref[ok])
    # decode(encode(decode(c))) == c for every finite code except -0 -> 0x80
    np.testing.assert_array_equal(C.e4m3fn_from_f32(got[ok]), codes[ok])


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(9)
    u = rng.integers(0, 1 << 32, 300_000, dtype=np.uint64).astype(np.uint32)
    # plus exact ties: low 16 bits 0x8000 with even and odd kept lsb
    ties = (rng.integers(0, 1 << 16, 2000, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    xs = np.concatenate([u, ties]).view(np.float32)
    ref = torch.from_numpy(xs).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = C.bf16_from_f32(xs)
    fin = ~np.isnan(xs)
    np.testing.assert_array_equal(got[fin], ref[fin])
    assert np.all((got[~fin] & 0x7FFF) > 0x7F80)  # NaN stays NaN


@pytest.mark.parametrize("mode", [1, 2, 3])
def test_quantisation_conventions(mode):
    """oracle/fp8.py (torch ops) == C restatement, on values that hit the
    clamp, subnormals and ties."""
    rng = np.random.default_rng(mode)
    x = np.concatenate([rng.standard_normal(20000) * 30, [1e4, -1e4, 0.0, 3e-4]]).astype(np.float32)
    x_bf16 = torch.from_numpy(x).to(torch.bfloat16)
    s = 0.0371
    if mode == 1:   # bf16 activations times a bf16 reciprocal scale
        s_t = torch.tensor([s], dtype=torch.bfloat16)
        ref = F.quantize_mul(x_bf16, s_t)
        s_c = float(s_t.float())
    elif mode == 2:  # fp32 product
        s_t = torch.tensor([s], dtype=torch.float32)
        ref = F.quantize_mul(x_bf16.float(), s_t)
        s_c = s
    else:            # fp32 division by the dequant scale
        s_t = torch.tensor([[s]], dtype=torch.float32)
        ref = F.quantize_div(x_bf16, s_t)
        s_c = s
    got = C.quantize_e4m3fn(x_bf16.float().numpy(), s_c, mode)
    np.testing.assert_array_equal(got, ref.view(torch.uint8).numpy())
