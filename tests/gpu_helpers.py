"""Shared helpers of the GPU parity tests (device buffers via torch, the
library via ctypes, the CPU oracle as the checker)."""
from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

import oracle
import vkblas_amd as vk
from vkblas_amd import hipblas_abi as hb

DEV = "cuda:0"


def to_dev(a: np.ndarray) -> torch.Tensor:
    """numpy (float32 or uint16 fp16 patterns) -> device tensor of the same bytes."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).view(torch.float16)
    else:
        t = torch.from_numpy(a)
    return t.to(DEV)


def to_host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype == torch.float16:
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()


def ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


def normwise(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got - ref| / max|ref| (0 if ref is all zero and got equals it)."""
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    d = np.max(np.abs(got - ref)) if got.size else 0.0
    s = np.max(np.abs(ref)) if ref.size else 0.0
    if s == 0.0:
        return float(d)
    return float(d / s)


def f32_bound(K: int) -> float:
    """north-star fp32 bound: relative error <= 1e-5 * sqrt(K)"""
    return 1e-5 * math.sqrt(K)


F16_BOUND = 2e-3
# bf16 results: kernel and oracle each round the same fp32-accurate value to
# bf16 once, so they differ by at most one bf16 ulp (2^-7 relative to the
# largest output) plus fp32 summation noise.
BF16_BOUND = 8e-3


class Handle:
    """A hipBLAS handle created through the library under test."""

    def __init__(self):
        self.abi = vk.hipblas()
        self.h = self.abi.create()

    def set_stream(self, stream_ptr):
        st = self.abi.hipblasSetStream(self.h, stream_ptr)
        assert st == hb.HIPBLAS_STATUS_SUCCESS

    def set_pointer_mode(self, mode):
        st = self.abi.hipblasSetPointerMode(self.h, mode)
        assert st == hb.HIPBLAS_STATUS_SUCCESS

    def close(self):
        if self.h is not None:
            self.abi.hipblasDestroy(self.h)
            self.h = None


def fbox(x: float):
    return ctypes.byref(ctypes.c_float(x))


def hbox(x: float):
    bits = int(np.array([x], dtype=np.float16).view(np.uint16)[0])
    return ctypes.byref(ctypes.c_uint16(bits))
