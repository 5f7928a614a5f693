"""GPU-side helpers for the parity tests: device buffers come from torch
(plumbing only); every computation goes through libtemplit_hip.so's C-ABI.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from templit_amd.native import NativeError, check, load_hip, u32_array


class Gpu:
    def __init__(self):
        if not torch.cuda.is_available():
            raise NativeError("no GPU visible: the HIP path cannot run here")
        self.lib = load_hip()
        check(self.lib.tlh_init(0), "tlh_init")
        self.stream = torch.cuda.current_stream().cuda_stream

    # -- buffers ---------------------------------------------------------------
    def dev(self, a: np.ndarray) -> torch.Tensor:
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint32:
            return torch.from_numpy(a.view(np.int32)).to("cuda")
        return torch.from_numpy(a.astype(np.float32, copy=False)).to("cuda")

    def dev_f64(self, a) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float64)).to("cuda")

    def empty(self, shape, dtype=torch.float32) -> torch.Tensor:
        return torch.empty(tuple(shape), dtype=dtype, device="cuda")

    def zeros(self, shape, dtype=torch.float32) -> torch.Tensor:
        return torch.zeros(tuple(shape), dtype=dtype, device="cuda")

    def host(self, t: torch.Tensor) -> np.ndarray:
        torch.cuda.synchronize()
        a = t.cpu().numpy()
        return a.view(np.uint32) if a.dtype == np.int32 else a

    def call(self, name: str, *args):
        fixed = []
        for a in args:
            if isinstance(a, torch.Tensor):
                fixed.append(a.data_ptr())
            elif isinstance(a, ctypes.Array):
                fixed.append(ctypes.addressof(a))
            else:
                fixed.append(a)
        check(getattr(self.lib, name)(*fixed, self.stream), name)

    def sync(self):
        torch.cuda.synchronize()


def u32(values):
    return u32_array(values)


def rel_err(a, b, floor: float = 1e-6) -> float:
    """max|a-b| / max(max|b|, floor); the floor keeps an exactly-zero
    expected result (e.g. dQ of a length-1 sequence) from dividing by 0."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), floor)) if b.size else 0.0


def assert_close(actual, expected, rtol=1e-4, atol=1e-5, what=""):
    """Element-wise |a-e| <= atol + rtol*|e| (the fp32 elementwise/reduction
    tolerance of the north star is rtol 1e-4, atol 1e-5)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, (what, a.shape, e.shape)
    with np.errstate(invalid="ignore"):
        bad = ~(np.abs(a - e) <= atol + rtol * np.abs(e))
    bad &= ~(np.isinf(a) & np.isinf(e) & (np.sign(a) == np.sign(e)))
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {bad.sum()} of {a.size} elements differ; first at {tuple(i)}: "
            f"got {a[tuple(i)]}, expected {e[tuple(i)]}")


def assert_rel(actual, expected, tol, what=""):
    """max|a-e| / max|e| <= tol (the matmul / attention tolerance, 1e-3)."""
    err = rel_err(actual, expected)
    assert err <= tol, f"{what}: relative error {err:.3e} > {tol}"
