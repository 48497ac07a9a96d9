/*
 * vkb_engine.h — internal entry of the host dispatcher (engine.c) for other
 * translation units of the library (not exported API).
 */
#pragma once
#include <stddef.h>
#include "vkblas_ext.h"

#ifdef __cplusplus
extern "C" {
#endif

/* vkblas_gemm_async with the split-K / decode partials in the caller's
 * device buffer `scratch` of `scratch_bytes` (at least 256-byte aligned):
 * allocates nothing.  A call whose partials need more than scratch_bytes
 * returns VKBLAS_ERR_PARAM before any launch. */
__attribute__((visibility("hidden")))
vkblas_status_t vkb_gemm_with_scratch(vkblas_dtype_t ab_type, vkblas_dtype_t c_type, vkblas_op_t op_a,
                                      vkblas_op_t op_b, uint32_t M, uint32_t N, uint32_t K, float alpha,
                                      const void* A, uint32_t lda, const void* B, uint32_t ldb, float beta,
                                      void* C, uint32_t ldc, uint32_t batch, int64_t stride_a, int64_t stride_b,
                                      int64_t stride_c, vkblas_scalar_mode_t scalar_mode, const void* alpha_dev,
                                      const void* beta_dev, uint32_t split_k, void* stream, void* scratch,
                                      size_t scratch_bytes);

#ifdef __cplusplus
}
#endif
