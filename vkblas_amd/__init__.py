"""vkblas_amd -- MI355X-native (gfx950) implementation of vkblas's GEMM hot path.

The product is ``libvkblas_hipblas.so`` in this directory: the reference's
public C API (``include/vkblas.h``), its hipBLAS ABI entry points (an
``LD_PRELOAD`` drop-in for PyTorch-ROCm) and the stream-aware extension
(``include/vkblas_ext.h``), all running hand-written gfx950 HIP kernels.

This module is the Python host-side binding used by the tests, the benchmark
and ``__graft_entry__``: it loads the built library with ctypes and mirrors the
engine entry points (``vkblas_gemm_f32`` / ``vkblas_gemm_f16`` of the
reference's ``src/vkblas.h:27-77``) with the same argument meaning and status
codes.  There is no fallback: if the library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
LIB_NAME = "libvkblas_hipblas.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
# the host dispatcher and kernels, opened by LIB_PATH's first call
ENGINE_PATH = os.path.join(HERE, "libvkblas_engine.so")

# vkblas_status_t (reference src/vkblas.h:6-12)
OK, ERR_INIT, ERR_IMPORT, ERR_PARAM, ERR_FALLBACK = 0, 1, 2, 3, 4
STATUS_NAMES = {0: "VKBLAS_OK", 1: "VKBLAS_ERR_INIT", 2: "VKBLAS_ERR_IMPORT", 3: "VKBLAS_ERR_PARAM",
                4: "VKBLAS_ERR_FALLBACK"}
# vkblas_op_t
OP_N, OP_T = 0, 1
# vkblas_dtype_t
DT_F32, DT_F16, DT_BF16 = 0, 1, 2
# vkblas_scalar_mode_t
SCALAR_HOST, SCALAR_DEV_F32, SCALAR_DEV_F16 = 0, 1, 2
# vkblas_path_t
PATH_NONE, PATH_TILE64, PATH_TILE128, PATH_TILE256, PATH_SPLITK, PATH_SKINNY, PATH_TAIL = range(7)
PATH_NAMES = {0: "none", 1: "tile64", 2: "tile128", 3: "tile256", 4: "splitk", 5: "skinny", 6: "tail"}


class VkblasError(RuntimeError):
    def __init__(self, status: int, what: str = "vkblas call"):
        super().__init__(f"{what} failed: {STATUS_NAMES.get(status, status)}")
        self.status = status


class Epilogue(ctypes.Structure):
    """vkblas_epilogue_t: C = alpha * op(A) op(B) + beta * c_in + bias[n]."""
    _fields_ = [("c_in", ctypes.c_void_p), ("ldc_in", ctypes.c_uint32), ("stride_c_in", ctypes.c_int64),
                ("bias", ctypes.c_void_p), ("bias_type", ctypes.c_int)]


class Plan(ctypes.Structure):
    _fields_ = [("path", ctypes.c_int), ("tile", ctypes.c_int), ("split", ctypes.c_uint32),
                ("k_per_split", ctypes.c_uint32), ("tail_rows", ctypes.c_uint32)]


_lib = None

_u32, _i64, _f, _vp, _int = ctypes.c_uint32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_int
_ENGINE_ARGS = [_int, _int, _u32, _u32, _u32, _f, _vp, _u32, _vp, _u32, _f, _vp, _u32, _u32, _i64, _i64, _i64]


def build(jobs: int = 8) -> None:
    """Compile every HIP kernel for gfx950 and link libvkblas_hipblas.so."""
    subprocess.run(["make", "-s", "-C", HERE, f"-j{jobs}", "-B"], check=True)


def load():
    """Load the built library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    for path in (LIB_PATH, ENGINE_PATH):
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run __graft_entry__.build() (make -C vkblas_amd)")
    L = ctypes.CDLL(LIB_PATH)
    for name in ("vkblas_gemm_f32", "vkblas_gemm_f16", "vkblas_gemm_bf16", "vkblas_gemm_bf16_hipblas"):
        fn = getattr(L, name)
        fn.argtypes = _ENGINE_ARGS
        fn.restype = _int
    L.vkblas_gemm_async.argtypes = [_int, _int, _int, _int, _u32, _u32, _u32, _f, _vp, _u32, _vp, _u32, _f, _vp,
                                    _u32, _u32, _i64, _i64, _i64, _int, _vp, _vp, _u32, _vp]
    L.vkblas_gemm_async.restype = _int
    L.vkblas_gemm_ex_async.argtypes = L.vkblas_gemm_async.argtypes[:-1] + [ctypes.POINTER(Epilogue), _vp]
    L.vkblas_gemm_ex_async.restype = _int
    L.vkblas_gemm_batched_async.argtypes = [_int, _int, _int, _int, _u32, _u32, _u32, _f, _vp, _u32, _vp, _u32, _f,
                                            _vp, _u32, _u32, _int, _vp, _vp, _vp]
    L.vkblas_gemm_batched_async.restype = _int
    L.vkblas_plan_gemm.argtypes = [_int, _int, _int, _int, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _u32, _int,
                                   ctypes.POINTER(Plan)]
    L.vkblas_plan_gemm.restype = _int
    L.vkblas_last_path.restype = _int
    L.vkblas_set_override.argtypes = [_int, _int]
    L.vkblas_set_override.restype = _int
    L.vkblas_version.restype = ctypes.c_char_p
    L.vkblas_cache_invalidate_base.argtypes = [_vp]
    L.vkblas_cache_invalidate_base.restype = None
    L.vkblas_last_kernel.restype = _int
    L.vkblas_workspace_release.restype = _int
    L.vkblas_gemm_noalloc_async.argtypes = L.vkblas_gemm_async.argtypes
    L.vkblas_gemm_noalloc_async.restype = _int
    L.vkblas_noalloc_scratch_bytes.restype = ctypes.c_size_t
    _lib = L
    return L


def version() -> str:
    return load().vkblas_version().decode()


def plan(ab_type, c_type, op_a, op_b, M, N, K, lda, ldb, ldc, batch=1, split_k=0, aligned=True) -> Plan:
    p = Plan()
    st = load().vkblas_plan_gemm(ab_type, c_type, op_a, op_b, M, N, K, lda, ldb, ldc, batch, split_k,
                                 1 if aligned else 0, ctypes.byref(p))
    if st != OK:
        raise VkblasError(st, "vkblas_plan_gemm")
    return p


def set_override(tile: int = -1, generic: bool = False) -> None:
    """Force a tile (-1 planner, 0: 64, 1: 128, 2: 256) / the generic kernel."""
    st = load().vkblas_set_override(tile, 1 if generic else 0)
    if st != OK:
        raise VkblasError(st, "vkblas_set_override")


def last_path() -> int:
    return load().vkblas_last_path()


# vkblas_kernel_t (include/vkblas_ext.h)
KERNEL_NONE, KERNEL_GENERIC, KERNEL_GENERIC_CHECKED, KERNEL_PIPE256, KERNEL_PIPE128, KERNEL_PIPE128_4, \
    KERNEL_SKINNY, KERNEL_WAVEK = range(8)


def workspace_release() -> None:
    """vkblas_workspace_release: free the per-stream partial buffers."""
    st = load().vkblas_workspace_release()
    if st != OK:
        raise VkblasError(st, "vkblas_workspace_release")


def last_kernel() -> int:
    """vkblas_kernel_t of the calling thread's most recent successful GEMM."""
    return load().vkblas_last_kernel()


def gemm_async(ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch=1,
               stride_a=0, stride_b=0, stride_c=0, scalar_mode=SCALAR_HOST, alpha_dev=None, beta_dev=None,
               split_k=0, stream=None, check=True) -> int:
    """vkblas_gemm_async on raw device pointers (ints).  Row-major engine
    contract of src/vkblas.h:21-26.  Returns the status (raises if check)."""
    st = load().vkblas_gemm_async(ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc,
                                  batch, stride_a, stride_b, stride_c, scalar_mode, alpha_dev, beta_dev, split_k,
                                  stream)
    if check and st != OK:
        raise VkblasError(st, "vkblas_gemm_async")
    return st


def gemm_ex_async(ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch=1,
                  stride_a=0, stride_b=0, stride_c=0, scalar_mode=SCALAR_HOST, alpha_dev=None, beta_dev=None,
                  split_k=0, c_in=None, ldc_in=0, stride_c_in=0, bias=None, bias_type=DT_F32, stream=None,
                  check=True) -> int:
    """vkblas_gemm_ex_async: gemm_async with a separate C input (c_in, beta's
    matrix) and a bias vector (one value per column n of C)."""
    ep = Epilogue(c_in, ldc_in, stride_c_in, bias, bias_type)
    st = load().vkblas_gemm_ex_async(ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc,
                                     batch, stride_a, stride_b, stride_c, scalar_mode, alpha_dev, beta_dev, split_k,
                                     ctypes.byref(ep), stream)
    if check and st != OK:
        raise VkblasError(st, "vkblas_gemm_ex_async")
    return st


def gemm_noalloc_async(ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch=1,
                       stride_a=0, stride_b=0, stride_c=0, scalar_mode=SCALAR_HOST, alpha_dev=None, beta_dev=None,
                       split_k=0, stream=None, check=True) -> int:
    """vkblas_gemm_noalloc_async: gemm_async with the partials in the library's
    per-device scratch array (allocates nothing)."""
    st = load().vkblas_gemm_noalloc_async(ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C,
                                          ldc, batch, stride_a, stride_b, stride_c, scalar_mode, alpha_dev, beta_dev,
                                          split_k, stream)
    if check and st != OK:
        raise VkblasError(st, "vkblas_gemm_noalloc_async")
    return st


def noalloc_scratch_bytes() -> int:
    return load().vkblas_noalloc_scratch_bytes()


def gemm_batched_async(ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch,
                       scalar_mode=SCALAR_HOST, alpha_dev=None, beta_dev=None, stream=None, check=True) -> int:
    """vkblas_gemm_batched_async: A, B, C are device addresses of arrays of
    `batch` matrix pointers (pointer-array batched GEMM)."""
    st = load().vkblas_gemm_batched_async(ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc,
                                          batch, scalar_mode, alpha_dev, beta_dev, stream)
    if check and st != OK:
        raise VkblasError(st, "vkblas_gemm_batched_async")
    return st


def gemm_f32(op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch=1, sa=0, sb=0, sc=0) -> int:
    """vkblas_gemm_f32 (reference src/vkblas.h:27-36); returns the status."""
    return load().vkblas_gemm_f32(op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch, sa, sb, sc)


def gemm_f16(op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch=1, sa=0, sb=0, sc=0) -> int:
    """vkblas_gemm_f16 (reference src/vkblas.h:68-77); returns the status."""
    return load().vkblas_gemm_f16(op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch, sa, sb, sc)


def gemm_bf16(op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch=1, sa=0, sb=0, sc=0) -> int:
    """vkblas_gemm_bf16 (reference src/vkblas.h:41-50); returns the status."""
    return load().vkblas_gemm_bf16(op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch, sa, sb, sc)


def gemm_bf16_hipblas(op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch=1, sa=0, sb=0, sc=0) -> int:
    """vkblas_gemm_bf16_hipblas (reference src/vkblas.h:55-64); returns the status."""
    return load().vkblas_gemm_bf16_hipblas(op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch, sa, sb,
                                           sc)


def hipblas():
    """The library's hipBLAS entry points, typed for ctypes callers."""
    from . import hipblas_abi
    return hipblas_abi.bind(load())
