"""ctypes binding of the bench-only MFMA rate probe (libvkblas_probe.so).

Not part of the drop-in library: bench.py's ``mfma_ceiling`` leg and its test
load it to measure the matrix rate the chip sustains for given operand data.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libvkblas_probe.so")
_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run make -C vkblas_amd")
        L = ctypes.CDLL(LIB_PATH)
        v, u = ctypes.c_void_p, ctypes.c_uint32
        L.vkblas_mfma_probe.argtypes = [ctypes.c_int, v, v, u, u, v]
        L.vkblas_mfma_probe.restype = ctypes.c_int
        _lib = L
    return _lib


def mfma_probe(bf16, operands, out, blocks, iters, stream=None) -> None:
    """blocks x 4 waves x iters x 32 v_mfma_f32_16x16x32 on the twelve
    fragments at `operands` (device pointer), no memory traffic; each thread
    writes one float to `out`."""
    st = load().vkblas_mfma_probe(1 if bf16 else 0, operands, out, blocks, iters, stream)
    if st != 0:
        raise RuntimeError(f"vkblas_mfma_probe: HIP error {st}")
