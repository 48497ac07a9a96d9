"""ctypes binding of the bench-only probes (libvkblas_probe.so): the MFMA
rate and the L2 -> LDS copy rate.

Not part of the drop-in library: bench.py's ``mfma_ceiling`` and
``copy_ceiling`` legs and their tests load it to measure the matrix rate the
chip sustains for given operand data and the rate a CU copies GEMM operand
tiles into LDS.
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
        L.vkblas_copy_probe.argtypes = [v, v, u, u, ctypes.c_int, ctypes.c_int, v, v]
        L.vkblas_copy_probe.restype = ctypes.c_int
        _lib = L
    return _lib


def mfma_probe(bf16, operands, out, blocks, iters, stream=None) -> None:
    """blocks x 4 waves x iters x 32 v_mfma_f32_16x16x32 on the twelve
    fragments at `operands` (device pointer), no memory traffic; each thread
    writes one float to `out`."""
    st = load().vkblas_mfma_probe(1 if bf16 else 0, operands, out, blocks, iters, stream)
    if st != 0:
        raise RuntimeError(f"vkblas_mfma_probe: HIP error {st}")


def copy_probe(A, B, n, blocks, steps_in_flight, row_bytes, out, stream=None) -> None:
    """blocks workgroups each copy the K steps of one 256 x 256 output tile's
    operands (A and B: n x n fp16, K-major, device pointers) into LDS by
    buffer_load ... lds, row_bytes (128 or 64) of each of the tile's 512 rows
    per step, steps_in_flight (1 or 2) steps of copies outstanding at each
    step's end; no compute.  out[b] (uint32, device pointer) receives the
    wrapping 32-bit sum of the words of workgroup b's last K step."""
    st = load().vkblas_copy_probe(A, B, n, blocks, steps_in_flight, row_bytes, out, stream)
    if st != 0:
        raise RuntimeError(f"vkblas_copy_probe: HIP error {st}")
