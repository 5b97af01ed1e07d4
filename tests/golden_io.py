"""Loader of the golden fixtures written by tests/golden/make_golden.py."""
import json
from pathlib import Path

import torch
from safetensors.torch import load_file

GOLDEN = Path(__file__).resolve().parent / "golden"


def load():
    meta = json.loads((GOLDEN / "attention_small.json").read_text())
    t = load_file(str(GOLDEN / "attention_small.safetensors"))
    return meta, t


def case(tensors, name, device="cpu"):
    """Tensors of one case with the name prefix stripped; uint8-stored fp8
    caches come back as float8_e4m3fn."""
    out = {}
    pre = name + "."
    for k, v in tensors.items():
        if not k.startswith(pre):
            continue
        k = k[len(pre):]
        if k.endswith("_u8"):
            k, v = k[:-3], v.view(torch.float8_e4m3fn)
        out[k] = v.to(device)
    return out
