"""Moving oracle storage arrays (numpy bit patterns) to and from the device."""
from __future__ import annotations

import numpy as np
import torch

import oracle as O

_TDT = {O.BF16: torch.bfloat16, O.F16: torch.float16, O.F32: torch.float32}


def to_dev(a: np.ndarray, dt: int, dev) -> torch.Tensor:
    if dt == O.F32:
        return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
    if dt in (O.BF16, O.F16):
        t = torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).to(dev)
        return t.view(_TDT[dt])
    if dt == O.U32:
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32)).to(dev)
    if dt == O.I32:
        return torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(dev)
    raise ValueError(dt)


def to_host(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def words_dev(a: np.ndarray, dev) -> torch.Tensor:
    """Packed u32 codes carried in an int32 tensor (same bits)."""
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).to(dev)


def tdtype(dt: int) -> torch.dtype:
    return _TDT[dt]
