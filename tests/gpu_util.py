"""Device-buffer helpers for the GPU parity tests (torch is plumbing only)."""
from __future__ import annotations

import numpy as np

_VIEW = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32,
         np.dtype(np.uint64): np.int64}


def dev(a: np.ndarray):
    """numpy array -> contiguous CUDA tensor with the same bytes."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype.fields is not None:
        a = a.view(np.uint8).reshape(-1)
    v = a.view(_VIEW.get(a.dtype, a.dtype))
    return torch.from_numpy(v.copy()).cuda()


def empty(n: int, dtype=np.uint16, fill=None):
    import torch
    tdt = {np.uint16: torch.int16, np.uint32: torch.int32, np.uint8: torch.uint8,
           np.float32: torch.float32}[dtype]
    t = torch.empty(n, dtype=tdt, device="cuda")
    if fill is not None:
        t.fill_(fill)
    return t


def host(t, dtype) -> np.ndarray:
    """CUDA tensor -> numpy array reinterpreted as `dtype`."""
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(dtype)


def f16_fill_bits(value: float) -> int:
    """fp16 bit pattern of `value` as a signed int16 (for tensor.fill_)."""
    b = int(np.array([value], np.float16).view(np.uint16)[0])
    return b - 65536 if b >= 32768 else b
