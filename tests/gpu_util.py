"""Helpers for GPU tests: numpy <-> device tensors (torch is only the allocator)."""
from __future__ import annotations

import sys

import numpy as np

_SIGNED = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32, np.dtype(np.uint64): np.int64}


def dev(arr: np.ndarray, device="cuda:0"):
    import torch
    arr = np.ascontiguousarray(arr)
    view = arr.view(_SIGNED.get(arr.dtype, arr.dtype))
    return torch.from_numpy(view.copy()).to(device)


def empty(shape, dtype, device="cuda:0"):
    import torch
    np_dtype = np.dtype(dtype)
    tdtype = {np.dtype(np.uint8): torch.uint8, np.dtype(np.int8): torch.int8,
              np.dtype(np.uint16): torch.int16, np.dtype(np.int16): torch.int16,
              np.dtype(np.int32): torch.int32, np.dtype(np.uint32): torch.int32,
              np.dtype(np.float32): torch.float32, np.dtype(np.float16): torch.float16,
              np.dtype(np.uint64): torch.int64, np.dtype(np.int64): torch.int64}[np_dtype]
    return torch.zeros(shape, dtype=tdtype, device=device)


def host(t, dtype=None) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    a = t.detach().cpu().numpy()
    if dtype is not None:
        a = a.view(dtype)
    return a


def say(*parts) -> None:
    """Names the case before a GPU step (flushed, so a crash still shows it)."""
    print("[gpu]", *parts, flush=True)
    sys.stdout.flush()
