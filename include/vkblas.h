/*
 * vkblas.h — public C API of the MI355X-native vkblas GEMM library.
 *
 * Every prototype below keeps the exact name, argument order and argument
 * types of the reference API (lakitu12/vkblas `src/vkblas.h`), so a program
 * that dlsym()s these symbols out of `libvkblas_hipblas.so` (the reference
 * tests do: `test/test_h.c:82-87`) binds to this library unchanged.
 *
 * Contract (reference `src/vkblas.h:21-26`), row-major:
 *     C[M,N] = alpha * A_eff[M,K] @ B_eff[K,N] + beta * C_old
 *     A_eff[m][k] = op_a == T ? A[k*lda + m] : A[m*lda + k]
 *     B_eff[k][n] = op_b == T ? B[n*ldb + k] : B[k*ldb + n]
 *   - A, B, C are HIP device pointers.
 *   - batch b uses A + b*stride_a, B + b*stride_b, C + b*stride_c (elements);
 *     a stride of 0 broadcasts one matrix to every batch, negative strides
 *     walk backwards.
 *   - beta == 0 never reads C (NaN/Inf already in C do not propagate).
 *   - M, N, K or batch == 0 returns VKBLAS_ERR_PARAM.
 *
 *   - Work runs on the HIP null stream and the call returns once C is
 *     written, as the reference's calls return after their Vulkan queue
 *     drains.  The asynchronous, stream-aware entry points are in
 *     vkblas_ext.h.
 *
 * Differences from the reference, all in the caller's favour:
 *   - Every transpose variant is computed natively; there is no hidden
 *     transposed copy and no dma-buf import cache.
 *   - fp16 accepts any ldc / N parity (the reference needed even ldc and N
 *     for its direct path).
 */
#pragma once
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Reference `src/vkblas.h:6-12`.  Values are part of the ABI. */
typedef enum {
    VKBLAS_OK = 0,
    VKBLAS_ERR_INIT,     /* no usable GPU / kernel image missing            */
    VKBLAS_ERR_IMPORT,   /* kept for ABI; this build has no import step      */
    VKBLAS_ERR_PARAM,    /* invalid argument (zero dims, bad ld, NULL ptr)   */
    VKBLAS_ERR_FALLBACK  /* kept for ABI; caller should loop or forward      */
} vkblas_status_t;

/* Reference `src/vkblas.h:14`. */
typedef enum { VKBLAS_OP_N = 0, VKBLAS_OP_T = 1 } vkblas_op_t;

/* Reference `src/vkblas.h:19`.  The reference dropped dma-buf imports of a
 * freed block here.  This build keeps no per-pointer state, so this is a
 * no-op that stays exported for ABI compatibility. */
void vkblas_cache_invalidate_base(const void* ptr);

/* fp32 GEMM, fp32 accumulate (MFMA v_mfma_f32_*_f32).
 * Replaces reference `src/vkblas.h:27-36` / `src/vkblas.c:3104-3341`. */
vkblas_status_t vkblas_gemm_f32(
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    float alpha,
    const void* A, uint32_t lda,
    const void* B, uint32_t ldb,
    float beta,
    void* C, uint32_t ldc,
    uint32_t batch,
    int64_t stride_a, int64_t stride_b, int64_t stride_c);

/* bf16 GEMM: A, B, C bf16; products and sums in fp32 (MFMA
 * v_mfma_f32_*_bf16); the result is rounded to bf16 once, to nearest even.
 * Reference `src/vkblas.h:41-50` / `src/vkblas.c:3345-3446`.  Runs on the
 * null stream and returns once C is written. */
vkblas_status_t vkblas_gemm_bf16(
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    float alpha,
    const void* A, uint32_t lda,
    const void* B, uint32_t ldb,
    float beta,
    void* C, uint32_t ldc,
    uint32_t batch,
    int64_t stride_a, int64_t stride_b, int64_t stride_c);

/* bf16 entry used by the reference's hipBLAS translation
 * (`src/vkblas.h:55-64`, `src/vkblas.c:3448-3512`).  Same contract and result
 * as vkblas_gemm_bf16 (the reference's variant differed only in an internal
 * transpose-avoidance choice). */
vkblas_status_t vkblas_gemm_bf16_hipblas(
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    float alpha,
    const void* A, uint32_t lda,
    const void* B, uint32_t ldb,
    float beta,
    void* C, uint32_t ldc,
    uint32_t batch,
    int64_t stride_a, int64_t stride_b, int64_t stride_c);

/* fp16 GEMM: A, B, C fp16; products and sums in fp32 (MFMA
 * v_mfma_f32_*_f16); the result is rounded to fp16 once, to nearest even.
 * Reference `src/vkblas.h:68-77` / `src/vkblas.c:3517-3651`. */
vkblas_status_t vkblas_gemm_f16(
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    float alpha,
    const void* A, uint32_t lda,
    const void* B, uint32_t ldb,
    float beta,
    void* C, uint32_t ldc,
    uint32_t batch,
    int64_t stride_a, int64_t stride_b, int64_t stride_c);

/* complex64 / fp64 / complex128 (reference `src/vkblas.h:82-118`).
 * Out of this build's scope: they return nonzero ("engine unavailable"),
 * which the reference documents as "caller forwards to the real library". */
int vkblas_gemm_c64(
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    float alpha_r, float alpha_i,
    const void* A, uint32_t lda,
    const void* B, uint32_t ldb,
    float beta_r, float beta_i,
    void* C, uint32_t ldc,
    uint32_t batch,
    int64_t stride_a, int64_t stride_b, int64_t stride_c);

int vkblas_gemm_f64(
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    double alpha,
    const void* A, uint32_t lda,
    const void* B, uint32_t ldb,
    double beta,
    void* C, uint32_t ldc,
    uint32_t batch,
    int64_t stride_a, int64_t stride_b, int64_t stride_c);

int vkblas_gemm_z64(
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    double alpha_r, double alpha_i,
    const void* A, uint32_t lda,
    const void* B, uint32_t ldb,
    double beta_r, double beta_i,
    void* C, uint32_t ldc,
    uint32_t batch,
    int64_t stride_a, int64_t stride_b, int64_t stride_c);

#ifdef __cplusplus
}
#endif
