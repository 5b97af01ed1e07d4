"""Small read-only device metadata (cu_seqlens, priors, identity tables) for
the functionals, made without host-to-device copies.

A blocking ``torch.tensor(..., device=...)`` copy is refused under HIP-graph
capture and costs a host sync per eager call; these helpers build the
tensor with device fill kernels instead and, in eager mode, keep it per
(device, values) for later calls.  Under ``torch.compile`` the tensor is a
graph constant (no cache: the compiled graph owns it); under stream capture
it is built in the graph and not cached (its memory belongs to the graph's
pool).
"""
from __future__ import annotations

from typing import Dict, Sequence, Tuple

import torch
from torch import Tensor

_CACHE: Dict[Tuple, Tensor] = {}
_MAX = 256


def _capturing(dev: torch.device) -> bool:
    return dev.type == "cuda" and torch.cuda.is_current_stream_capturing()


def device_i32(dev: torch.device, values: Sequence[int]) -> Tensor:
    """int32 ``[len(values)]`` on ``dev`` (read-only: callers never write it)."""
    values = tuple(int(v) for v in values)
    if torch.compiler.is_compiling():
        return torch.tensor(values, dtype=torch.int32, device=dev)
    key = ("v", str(dev), values)
    t = _CACHE.get(key)
    if t is not None:
        return t
    t = torch.empty(len(values), dtype=torch.int32, device=dev)
    for i, v in enumerate(values):
        t[i:i + 1].fill_(v)
    if not _capturing(dev):
        if len(_CACHE) >= _MAX:
            _CACHE.clear()
        _CACHE[key] = t
    return t


def identity_table(dev: torch.device, nblk: int) -> Tensor:
    """Block table ``[1, nblk]`` = ``0 .. nblk-1`` (int32, read-only)."""
    if torch.compiler.is_compiling():
        return torch.arange(nblk, dtype=torch.int32, device=dev).view(1, nblk)
    key = ("id", str(dev), int(nblk))
    t = _CACHE.get(key)
    if t is None:
        t = torch.arange(nblk, dtype=torch.int32, device=dev).view(1, nblk)
        if not _capturing(dev):
            if len(_CACHE) >= _MAX:
                _CACHE.clear()
            _CACHE[key] = t
    return t
