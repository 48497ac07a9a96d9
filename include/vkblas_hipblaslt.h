/*
 * vkblas_hipblaslt.h — the hipBLASLt entry points exported by
 * libvkblas_hipblas.so.
 *
 * PyTorch-ROCm on gfx950 computes its matrix products (mm, bmm, addmm and
 * linear with a 1-D bias) through hipblasLtMatmul by default, bypassing
 * hipBLAS and rocBLAS, so an LD_PRELOAD drop-in has to interpose this layer
 * too; the reference met the same kind of bypass by interposing the layer
 * PyTorch actually called (src/vkblas_hipblas.c:802-808).  Signatures are
 * hipBLASLt 1.x (ROCm 7.2); the shim includes this header after
 * <hipblaslt/hipblaslt.h> (a C++ header), so the compiler checks every
 * declaration against the vendor's.
 *
 * hipblasLtMatmul is computed by this library for column-major A, B, C, D of
 * (fp32, fp32 -> fp32 / fp16 / bf16), (fp16, fp16 -> fp16 / fp32) and
 * (bf16, bf16 -> bf16 / fp32) with fp32 scale type and a 32-bit float compute
 * type, epilogue HIPBLASLT_EPILOGUE_DEFAULT or HIPBLASLT_EPILOGUE_BIAS (an
 * fp32 / fp16 / bf16 bias vector of D's row count), host or device alpha /
 * beta, a D separate from C, and equal batch counts with any strides.
 * Everything else (scale pointers, fp8, activation and gradient epilogues,
 * other orders) is forwarded to the real hipBLASLt of the process.  What a
 * matmul descriptor or a matrix layout holds cannot be read back through the
 * hipBLASLt API (PyTorch's bundled hipBLASLt answers only a layout's batch
 * count and stride; no call gives a descriptor's compute and scale types),
 * so their create / set-attribute / destroy calls are interposed too: each
 * is forwarded to the real library unchanged and recorded when it succeeds.
 */
#pragma once
#include <hipblaslt/hipblaslt.h>

#ifdef __cplusplus
extern "C" {
#endif

hipblasStatus_t hipblasLtMatmulDescCreate(hipblasLtMatmulDesc_t* matmulDesc, hipblasComputeType_t computeType,
                                          hipDataType scaleType);

hipblasStatus_t hipblasLtMatmulDescDestroy(const hipblasLtMatmulDesc_t matmulDesc);

hipblasStatus_t hipblasLtMatmulDescSetAttribute(hipblasLtMatmulDesc_t matmulDesc,
                                                hipblasLtMatmulDescAttributes_t attr, const void* buf,
                                                size_t sizeInBytes);

hipblasStatus_t hipblasLtMatrixLayoutCreate(hipblasLtMatrixLayout_t* matLayout, hipDataType type, uint64_t rows,
                                            uint64_t cols, int64_t ld);

hipblasStatus_t hipblasLtMatrixLayoutDestroy(const hipblasLtMatrixLayout_t matLayout);

hipblasStatus_t hipblasLtMatrixLayoutSetAttribute(hipblasLtMatrixLayout_t matLayout,
                                                  hipblasLtMatrixLayoutAttribute_t attr, const void* buf,
                                                  size_t sizeInBytes);

hipblasStatus_t hipblasLtMatmul(hipblasLtHandle_t handle, hipblasLtMatmulDesc_t matmulDesc, const void* alpha,
                                const void* A, hipblasLtMatrixLayout_t Adesc, const void* B,
                                hipblasLtMatrixLayout_t Bdesc, const void* beta, const void* C,
                                hipblasLtMatrixLayout_t Cdesc, void* D, hipblasLtMatrixLayout_t Ddesc,
                                const hipblasLtMatmulAlgo_t* algo, void* workspace, size_t workspaceSizeInBytes,
                                hipStream_t stream);

#ifdef __cplusplus
}
#endif
