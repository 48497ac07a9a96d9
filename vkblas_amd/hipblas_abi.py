"""ctypes typing of the hipBLAS entry points exported by libvkblas_hipblas.so.

Mirrors how the reference's C tests bind the shim: ``dlopen`` the library and
``dlsym`` the hipBLAS symbols (``test/test_gemm.c:210-219``,
``test/test_v9h.c:50-52``).  Enum values are hipBLAS 3.x / hipDataType ones.
"""
from __future__ import annotations

import ctypes

# hipblasOperation_t
HIPBLAS_OP_N, HIPBLAS_OP_T, HIPBLAS_OP_C = 111, 112, 113
# hipblasStatus_t
HIPBLAS_STATUS_SUCCESS, HIPBLAS_STATUS_INVALID_VALUE, HIPBLAS_STATUS_NOT_SUPPORTED = 0, 3, 7
# hipblasPointerMode_t
HIPBLAS_POINTER_MODE_HOST, HIPBLAS_POINTER_MODE_DEVICE = 0, 1
# hipDataType
HIP_R_32F, HIP_R_16F, HIP_R_16BF = 0, 2, 14
# hipblasComputeType_t
HIPBLAS_COMPUTE_16F, HIPBLAS_COMPUTE_32F = 0, 2
HIPBLAS_GEMM_DEFAULT = 160

_vp, _i, _ll, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_size_t

_SIGS = {
    "hipblasCreate": [ctypes.POINTER(_vp)],
    "hipblasDestroy": [_vp],
    "hipblasSetStream": [_vp, _vp],
    "hipblasGetStream": [_vp, ctypes.POINTER(_vp)],
    "hipblasSetPointerMode": [_vp, _i],
    "hipblasGetPointerMode": [_vp, ctypes.POINTER(_i)],
    "hipblasSetWorkspace": [_vp, _vp, _sz],
    # (handle, transA, transB, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    "hipblasSgemm": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp, _i, _vp, _vp, _i],
    "hipblasHgemm": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp, _i, _vp, _vp, _i],
    "hipblasSgemmStridedBatched": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _ll, _vp, _i, _ll, _vp, _vp, _i, _ll, _i],
    "hipblasHgemmStridedBatched": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _ll, _vp, _i, _ll, _vp, _vp, _i, _ll, _i],
    # (handle, tA, tB, m, n, k, alpha, A, aType, lda, B, bType, ldb, beta, C, cType, ldc, compute, algo)
    "hipblasGemmEx": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp, _i, _i, _vp, _vp, _i, _i, _i, _i],
    "hipblasGemmEx_v2": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp, _i, _i, _vp, _vp, _i, _i, _i, _i],
    "hipblasGemmStridedBatchedEx": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _ll, _vp, _i, _i, _ll, _vp, _vp, _i,
                                    _i, _ll, _i, _i, _i],
    "hipblasGemmStridedBatchedEx_v2": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _ll, _vp, _i, _i, _ll, _vp, _vp,
                                       _i, _i, _ll, _i, _i, _i],
    # pointer-array batched: A, B, C are device arrays of matrix pointers
    # (handle, tA, tB, m, n, k, alpha, A[], lda, B[], ldb, beta, C[], ldc, batch)
    "hipblasSgemmBatched": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp, _i, _vp, _vp, _i, _i],
    "hipblasHgemmBatched": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _vp, _i, _vp, _vp, _i, _i],
    # (handle, tA, tB, m, n, k, alpha, A[], aType, lda, B[], bType, ldb, beta, C[], cType, ldc, batch, compute,
    #  algo)
    "hipblasGemmBatchedEx": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp, _i, _i, _vp, _vp, _i, _i, _i, _i, _i],
}


class HipblasABI:
    def __init__(self, lib):
        self.lib = lib
        for name, args in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = _i
            setattr(self, name, fn)

    def create(self):
        h = _vp()
        st = self.hipblasCreate(ctypes.byref(h))
        if st != HIPBLAS_STATUS_SUCCESS:
            raise RuntimeError(f"hipblasCreate failed: {st}")
        return h


_bound = None


def bind(lib) -> HipblasABI:
    global _bound
    if _bound is None or _bound.lib is not lib:
        _bound = HipblasABI(lib)
    return _bound


def exported_names() -> list:
    return sorted(_SIGS)
