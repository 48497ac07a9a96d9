"""CPU oracle for the vkblas GEMM hot path (test infrastructure).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed CPU
comparator.  The library under test never calls it and has no CPU fallback.

The arithmetic lives in ``ref_gemm.c`` (built into ``liboracle.so`` by
``oracle/Makefile``); each C function cites the reference code it restates:

* ``ref_gemm_cm``      -- ``test/test_gemm.c:32-58`` (hipBLAS column-major,
  double accumulation, ``alpha*(float)s + beta*C``, optional row sampling);
* ``fill_test_gemm``   -- ``test/test_gemm.c:70-73`` (glibc ``srand(seed)``,
  ``(rand()%200-100)/10``);
* ``ref_gemm_f16_rm``  -- ``test/test_h.c:63-79`` (row-major fp16, double
  accumulation, one fp16 rounding, to nearest even);
* ``fill_test_h``      -- ``test/test_h.c:102,111-113``;
* ``ref_gemm_f32_rm``  -- the row-major engine contract ``src/vkblas.h:21-26``;
* ``f2bf_rne`` / ``bf2f`` -- bf16 conversions of
  ``src/shaders/gemm_half_128x128_bankfree_tmpl.comp:26-47``;
* ``ref_gemm_bf16_rm`` -- ``src/vkblas.c:3345-3512`` (bf16 in, fp32
  arithmetic, one bf16 rounding) on the row-major engine contract;
* ``ref_gemm_tiled_rm`` -- the same arithmetic as ``ref_gemm_epi_rm`` in
  cache-sized tiles, bit for bit equal to it, for whole-output checks of large
  shapes.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float


def build() -> None:
    """Compile liboracle.so from ref_gemm.c (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_h2f.restype = ctypes.c_float
        L.oracle_h2f.argtypes = [ctypes.c_uint16]
        L.oracle_f2h_rne.restype = ctypes.c_uint16
        L.oracle_f2h_rne.argtypes = [ctypes.c_float]
        L.oracle_f2h_ties_away.restype = ctypes.c_uint16
        L.oracle_f2h_ties_away.argtypes = [ctypes.c_float]
        L.oracle_f2h_rne_array.argtypes = [_f32p, _u16p, _i64]
        L.oracle_f2bf_rne_array.argtypes = [_f32p, _u16p, _i64]
        L.oracle_bf2f_array.argtypes = [_u16p, _f32p, _i64]
        L.oracle_h2f_array.argtypes = [_u16p, _f32p, _i64]
        L.oracle_fill_test_gemm.argtypes = [ctypes.c_uint, _f32p, _i64, _f32p, _i64, _f32p, _i64]
        L.oracle_fill_test_h.argtypes = [ctypes.c_uint, _u16p, _i64, _u16p, _i64, _u16p, _i64]
        L.oracle_sample_rows.argtypes = [_int, _int, _i32p]
        L.oracle_sample_rows.restype = _int
        cm = [_int, _int, _int, _int, _int, _flt, _f32p, _i64, _f32p, _i64, _flt, _f32p, _i64, _int]
        L.oracle_ref_gemm_cm.argtypes = cm
        L.oracle_ref_gemm_cm_omp.argtypes = cm + [_int]
        rows_t = ctypes.c_void_p
        L.oracle_ref_gemm_f16_rm.argtypes = [_int, _int, _int, _int, _int, _u16p, _i64, _u16p, _i64, _flt, _flt,
                                             _u16p, _i64, rows_t, _int, _int]
        L.oracle_ref_gemm_f16f32_rm.argtypes = [_int, _int, _int, _int, _int, _u16p, _i64, _u16p, _i64, _flt,
                                                _flt, _f32p, _i64, rows_t, _int, _int]
        for nm in ("oracle_ref_gemm_bf16_rm",):
            getattr(L, nm).argtypes = L.oracle_ref_gemm_f16_rm.argtypes
        L.oracle_ref_gemm_bf16f32_rm.argtypes = L.oracle_ref_gemm_f16f32_rm.argtypes
        L.oracle_ref_gemm_f32_rm.argtypes = [_int, _int, _int, _int, _int, _f32p, _i64, _f32p, _i64, _flt, _flt,
                                             _f32p, _i64, rows_t, _int, _int]
        _vp = ctypes.c_void_p
        L.oracle_ref_gemm_epi_rm.argtypes = [_int, _int, _int, _int, _int, _int, _int, _vp, _i64, _vp, _i64, _flt,
                                             _flt, _vp, _i64, _vp, _i64, _vp, rows_t, _int, _int]
        L.oracle_ref_gemm_tiled_rm.argtypes = [_int, _int, _int, _int, _int, _int, _int, _vp, _i64, _vp, _i64,
                                               _flt, _flt, _vp, _i64, _int]
        _lib = L
    return _lib


# ----------------------------------------------------------------- fp16 bits

def f2h_rne(x) -> np.ndarray:
    """float32 array -> fp16 bit patterns (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f2h_rne_array(x.reshape(-1), y.reshape(-1), x.size)
    return y


def h2f(h) -> np.ndarray:
    """fp16 bit patterns (uint16) -> float32."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().oracle_h2f_array(h.reshape(-1), y.reshape(-1), h.size)
    return y


def f2bf_rne(x) -> np.ndarray:
    """float32 array -> bf16 bit patterns (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f2bf_rne_array(x.reshape(-1), y.reshape(-1), x.size)
    return y


def bf2f(h) -> np.ndarray:
    """bf16 bit patterns (uint16) -> float32."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().oracle_bf2f_array(h.reshape(-1), y.reshape(-1), h.size)
    return y


# --------------------------------------------------------------- generators

def fill_test_gemm(seed: int, na: int, nb: int, nc: int):
    """Inputs of a test_gemm.c case: A, B, C float32 from glibc rand()."""
    A = np.empty(na, np.float32)
    B = np.empty(nb, np.float32)
    C = np.empty(nc, np.float32)
    lib().oracle_fill_test_gemm(seed, A, na, B, nb, C, nc)
    return A, B, C


def fill_test_h(seed: int, na: int, nb: int, nc: int):
    """Inputs of a test_h.c fp16 case: uint16 fp16 patterns of U[-1,1)."""
    A = np.empty(na, np.uint16)
    B = np.empty(nb, np.uint16)
    C = np.empty(nc, np.uint16)
    lib().oracle_fill_test_h(seed, A, na, B, nb, C, nc)
    return A, B, C


def sample_rows(m: int, sample: int) -> np.ndarray:
    rows = np.empty(max(m, 1), np.int32)
    n = lib().oracle_sample_rows(m, sample, rows)
    return rows[:n].copy()


# ------------------------------------------------------------------ GEMMs

def ref_gemm_cm(ta: int, tb: int, m: int, n: int, k: int, alpha: float, A, lda: int, B, ldb: int,
                beta: float, C, ldc: int, sample: int = 0, threads: int = 1) -> None:
    """test_gemm.c ref_gemm, in place on C (float32, column-major buffers)."""
    if threads == 1:
        lib().oracle_ref_gemm_cm(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, sample)
    else:
        lib().oracle_ref_gemm_cm_omp(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, sample, threads)


def _rows_arg(rows):
    if rows is None:
        return None, 0, None
    r = np.ascontiguousarray(rows, dtype=np.int32)
    return r.ctypes.data_as(ctypes.c_void_p), len(r), r


def ref_gemm_f16_rm(op_a: int, op_b: int, M: int, N: int, K: int, A, lda: int, B, ldb: int,
                    alpha: float, beta: float, C, ldc: int, rows=None, threads: int = 0) -> None:
    """test_h.c cpu_ref (fp16), in place on C (uint16 fp16 patterns, row-major)."""
    p, n, keep = _rows_arg(rows)
    lib().oracle_ref_gemm_f16_rm(op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, ldc, p, n, threads)
    del keep


def ref_gemm_f16f32_rm(op_a: int, op_b: int, M: int, N: int, K: int, A, lda: int, B, ldb: int,
                       alpha: float, beta: float, C, ldc: int, rows=None, threads: int = 0) -> None:
    """fp16 inputs, fp32 result, in place on C (float32, row-major)."""
    p, n, keep = _rows_arg(rows)
    lib().oracle_ref_gemm_f16f32_rm(op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, ldc, p, n, threads)
    del keep


def ref_gemm_f32_rm(op_a: int, op_b: int, M: int, N: int, K: int, A, lda: int, B, ldb: int,
                    alpha: float, beta: float, C, ldc: int, rows=None, threads: int = 0) -> None:
    """fp32 engine contract (row-major, beta == 0 never reads C), in place on C."""
    p, n, keep = _rows_arg(rows)
    lib().oracle_ref_gemm_f32_rm(op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, ldc, p, n, threads)
    del keep


def ref_gemm_bf16_rm(op_a: int, op_b: int, M: int, N: int, K: int, A, lda: int, B, ldb: int,
                     alpha: float, beta: float, C, ldc: int, rows=None, threads: int = 0) -> None:
    """bf16 GEMM (vkblas_gemm_bf16), in place on C (uint16 bf16 patterns, row-major)."""
    p, n, keep = _rows_arg(rows)
    lib().oracle_ref_gemm_bf16_rm(op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, ldc, p, n, threads)
    del keep


_TCODE = {"f32": 0, "f16": 1, "bf16": 2}


def ref_gemm_epi_rm(ab: str, ct: str, op_a: int, op_b: int, M: int, N: int, K: int, A, lda: int, B, ldb: int,
                    alpha: float, beta: float, Cin, ldcin: int, D, ldd: int, bias=None, rows=None,
                    threads: int = 0) -> None:
    """D = alpha * A.B + beta * Cin + bias[n] (hipBLASLt bias epilogue, separate C and D), one rounding to
    D's type.  ab / ct: "f32", "f16" or "bf16" (16-bit data as uint16 bit patterns); bias: float32 values
    or None.  In place on D (row-major)."""
    p, n, keep = _rows_arg(rows)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().oracle_ref_gemm_epi_rm(_TCODE[ab], _TCODE[ct], op_a, op_b, M, N, K, A.ctypes.data, lda, B.ctypes.data,
                                 ldb, alpha, beta, Cin.ctypes.data, ldcin, D.ctypes.data, ldd,
                                 None if b is None else b.ctypes.data, p, n, threads)
    del keep


def ref_gemm_bf16f32_rm(op_a: int, op_b: int, M: int, N: int, K: int, A, lda: int, B, ldb: int,
                        alpha: float, beta: float, C, ldc: int, rows=None, threads: int = 0) -> None:
    """bf16 inputs, fp32 result (GemmEx 16BF -> 32F), in place on C (float32, row-major)."""
    p, n, keep = _rows_arg(rows)
    lib().oracle_ref_gemm_bf16f32_rm(op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, ldc, p, n, threads)
    del keep


def ref_gemm_tiled_rm(ab: str, ct: str, op_a: int, op_b: int, M: int, N: int, K: int, A, lda: int, B, ldb: int,
                      alpha: float, beta: float, C, ldc: int, threads: int = 0) -> None:
    """The whole output of ref_gemm_epi_rm (no bias, C_in == C), bit for bit, computed in cache-sized tiles:
    for full-output checks of large shapes.  ab / ct: "f32", "f16" or "bf16"; in place on C (row-major)."""
    lib().oracle_ref_gemm_tiled_rm(_TCODE[ab], _TCODE[ct], op_a, op_b, M, N, K, A.ctypes.data, lda, B.ctypes.data,
                                   ldb, alpha, beta, C.ctypes.data, ldc, threads)
