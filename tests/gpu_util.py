"""Helpers for the GPU parity tests (test infrastructure)."""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import torch

_hip = None


def note(msg: str) -> None:
    """Name the case about to run on the GPU, flushed before the launch."""
    print(f"[gpu] {msg}", file=sys.stderr, flush=True)


def hip():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipMemcpy.restype = ctypes.c_int
    return _hip


def read_f16(ptr: int, offset_elems: int, n: int) -> np.ndarray:
    """Copy n f16 values at device address ptr + 2*offset to host (as f32)."""
    out = np.empty(n, np.float16)
    rc = hip().hipMemcpy(out.ctypes.data, ptr + 2 * offset_elems, 2 * n, 2)
    assert rc == 0, f"hipMemcpy failed: {rc}"
    return out.astype(np.float32)


def read_f32(ptr: int, offset_elems: int, n: int) -> np.ndarray:
    """Copy n f32 values at device address ptr + 4*offset to host."""
    out = np.empty(n, np.float32)
    rc = hip().hipMemcpy(out.ctypes.data, ptr + 4 * offset_elems, 4 * n, 2)
    assert rc == 0, f"hipMemcpy failed: {rc}"
    return out


def dev(x: np.ndarray, dtype=torch.float32) -> torch.Tensor:
    """Host float32 array (values exact in dtype) -> contiguous device tensor."""
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.detach().float().cpu().numpy()


def maxerr(a, b) -> float:
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max())
