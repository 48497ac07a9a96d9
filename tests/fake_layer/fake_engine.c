/*
 * fake_engine.c — a stand-in for libvkblas_engine.so used by the CPU tests of
 * the drop-in library's failure path.  Every GEMM entry point records its
 * call and returns the status named by FAKE_ENGINE_STATUS (default
 * VKBLAS_ERR_INIT, "engine unavailable"); nothing touches a GPU.  The
 * reference forwards to the real hipBLAS when its engine fails
 * (src/vkblas_hipblas.c:244-246, 268-271); the drop-in must do the same.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "vkblas_ext.h"

static int g_calls;
static uint32_t g_last[3];   /* M, N, K as the engine saw them */

static vkblas_status_t fake_status(void) {
    const char* e = getenv("FAKE_ENGINE_STATUS");
    return e ? (vkblas_status_t)atoi(e) : VKBLAS_ERR_INIT;
}

int fake_engine_calls(void) { return g_calls; }
void fake_engine_last(uint32_t* mnk) { memcpy(mnk, g_last, sizeof(g_last)); }

#define REC(M_, N_, K_) (++g_calls, g_last[0] = (M_), g_last[1] = (N_), g_last[2] = (K_), fake_status())

vkblas_status_t vkblas_gemm_async(vkblas_dtype_t ab_type, vkblas_dtype_t c_type, vkblas_op_t op_a, vkblas_op_t op_b,
                                  uint32_t M, uint32_t N, uint32_t K, float alpha, const void* A, uint32_t lda,
                                  const void* B, uint32_t ldb, float beta, void* C, uint32_t ldc, uint32_t batch,
                                  int64_t stride_a, int64_t stride_b, int64_t stride_c,
                                  vkblas_scalar_mode_t scalar_mode, const void* alpha_dev, const void* beta_dev,
                                  uint32_t split_k, void* stream) {
    return REC(M, N, K);
}

vkblas_status_t vkblas_gemm_ex_async(vkblas_dtype_t ab_type, vkblas_dtype_t c_type, vkblas_op_t op_a,
                                     vkblas_op_t op_b, uint32_t M, uint32_t N, uint32_t K, float alpha,
                                     const void* A, uint32_t lda, const void* B, uint32_t ldb, float beta, void* C,
                                     uint32_t ldc, uint32_t batch, int64_t stride_a, int64_t stride_b,
                                     int64_t stride_c, vkblas_scalar_mode_t scalar_mode, const void* alpha_dev,
                                     const void* beta_dev, uint32_t split_k, const vkblas_epilogue_t* epilogue,
                                     void* stream) {
    return REC(M, N, K);
}

vkblas_status_t vkblas_gemm_batched_async(vkblas_dtype_t ab_type, vkblas_dtype_t c_type, vkblas_op_t op_a,
                                          vkblas_op_t op_b, uint32_t M, uint32_t N, uint32_t K, float alpha,
                                          const void* const* A, uint32_t lda, const void* const* B, uint32_t ldb,
                                          float beta, void* const* C, uint32_t ldc, uint32_t batch,
                                          vkblas_scalar_mode_t scalar_mode, const void* alpha_dev,
                                          const void* beta_dev, void* stream) {
    return REC(M, N, K);
}

const char* vkblas_version(void) { return "fake engine"; }
