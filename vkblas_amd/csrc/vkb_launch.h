/*
 * vkb_launch.h — internal C ABI between the host dispatcher (engine.c, C11)
 * and the gfx950 HIP kernels (*.hip).  Plain pointers, sizes and scalars
 * only; every launcher enqueues on the given stream and returns 0 on success
 * or a hipError_t value.
 *
 * Operand convention (row-major engine contract, reference src/vkblas.h:21-26):
 *   C[M,N] = alpha * A_eff[M,K] @ B_eff[K,N] + beta * C
 *   a_kmajor = (op_a == N): A row m is K-contiguous  (A[m*lda + k])
 *              otherwise     A column is M-contiguous (A[k*lda + m])
 *   b_kmajor = (op_b == T): B row n is K-contiguous  (B[n*ldb + k])
 *              otherwise     B row k is N-contiguous  (B[k*ldb + n])
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types (values match vkblas_dtype_t in vkblas_ext.h) */
enum { VKB_T_F32 = 0, VKB_T_F16 = 1, VKB_T_BF16 = 2 };

/* how alpha / beta reach the kernel */
enum { VKB_SCALAR_HOST = 0, VKB_SCALAR_DEV_F32 = 1, VKB_SCALAR_DEV_F16 = 2 };

/* GEMM kernel that ran (vkb_gemm_args.kernel_out, vkblas_last_kernel) */
enum {
    VKB_KERN_NONE = 0,
    VKB_KERN_GENERIC = 1,          /* gemm_kernel<>, full tiles             */
    VKB_KERN_GENERIC_CHECKED = 2,  /* gemm_kernel<>, edge handling          */
    VKB_KERN_PIPE256 = 3,          /* gemm_pipe_kernel, 256x256 tiles       */
    VKB_KERN_PIPE128 = 4,          /* gemm_pipe_kernel, 128x128, 2 stages   */
    VKB_KERN_PIPE128_4 = 5,        /* gemm_pipe_kernel, 128x128, 4 stages   */
    VKB_KERN_SKINNY = 6,           /* decode kernels (skinny.hip)           */
    VKB_KERN_WAVEK = 7             /* gemm_wavek_kernel: split-K pass 1 on
                                      32x32 / 64x64 tiles, K over the waves */
};

/* GEMM tile configurations (block tile BM x BN, 4 waves, BK = 128 bytes) */
enum {
    VKB_TILE_64  = 0,  /*  64 x  64, waves 2x2 of  32x32 */
    VKB_TILE_128 = 1,  /* 128 x 128, waves 2x2 of  64x64 */
    VKB_TILE_256 = 2,  /* 256 x 256, waves 2x2 of 128x128 */
    VKB_TILE_COUNT = 3,
    VKB_TILE_32 = 3,   /* 32 x 32, split-K pass 1 only (gemm_wavek_kernel:
                          each wave the whole tile over a quarter of the
                          slice's K); not a choice for unsplit GEMMs */
    VKB_TILE_64Q = 4   /* 64 x 64, split-K pass 1 only (gemm_wavek_kernel),
                          each K slice divided among VKB_WAVEK_NQ workgroups
                          per output tile whose sums the last of them to
                          finish adds in a fixed order (vkb_gemm_args.qpart) */
};

/* Workgroups sharing one K slice of a 64 x 64 tile under VKB_TILE_64Q. */
#define VKB_WAVEK_NQ 4
/* Every partials workspace (split-K, split decode) starts with this many
 * bytes of 32-bit arrival counters for VKB_TILE_64Q, zeroed when the
 * workspace is allocated; the partials follow.  Each VKB_TILE_64Q launch
 * adds VKB_WAVEK_NQ to every counter it uses, so they stay multiples of it. */
#define VKB_WS_HEADER 4096u
#define VKB_WS_COUNTERS (VKB_WS_HEADER / 4u)

/* Optional epilogue inputs (every launcher):
 *   C = alpha * acc + beta * C_in + bias[n]
 * c_in: the matrix beta scales, of the output's element type, with its own
 *       leading dimension and batch stride; NULL = C itself (in place).
 *       Read only when beta != 0.
 * bias: NULL, or one value per column n of C (bias_type: VKB_T_*), shared by
 *       every batch, added after alpha / beta and before the one rounding. */
typedef struct vkb_epilogue_args {
    const void* c_in;
    int64_t ldc_in;
    int64_t stride_c_in;
    const void* bias;
    int bias_type;
} vkb_epilogue_args;

typedef struct vkb_gemm_args {
    const void* A;
    const void* B;
    void* C;
    int64_t lda, ldb, ldc;
    int64_t stride_a, stride_b, stride_c;  /* per batch, elements */
    uint32_t M, N, K;
    uint32_t batch;
    /* split-K pass 1: split > 1 writes raw fp32 partial sums of K-slice s
     * (k in [s*k_per_split, min(K,(s+1)*k_per_split))) to
     * C + s*stride_split with alpha = 1, beta = 0. */
    uint32_t split;
    uint32_t k_per_split;
    int64_t stride_split;
    int a_kmajor, b_kmajor;
    int ab_type, c_type;
    float alpha, beta;
    int scalar_mode;
    const void* alpha_dev;
    const void* beta_dev;
    /* 0: best kernel for the shape; 1: always the generic blocked kernel */
    int generic_only;
    /* 1: A, B, C are device arrays of `batch` matrix pointers (stride_* are
     * unused); runs the checked generic kernel, split must be 1 */
    int ptr_array;
    /* optional: receives the VKB_KERN_* value of the launched kernel */
    int* kernel_out;
    /* optional epilogue inputs (NULL: in place, no bias); unused by split-K
     * pass 1, whose raw partials take no epilogue */
    const vkb_epilogue_args* epi;
    /* tile VKB_TILE_64Q only: the VKB_WAVEK_NQ workgroups of a (slice, tile)
     * store their 64 x 64 sums to qpart + ((slice * tiles + tile) * NQ + q)
     * * 4096 floats and count their arrival in qcnt[slice * tiles + tile]
     * (at most VKB_WS_COUNTERS words, each a multiple of NQ at launch); the
     * last to arrive writes the slice's partial to C. */
    float* qpart;
    uint32_t* qcnt;
} vkb_gemm_args;

/* Tile-config properties the dispatcher plans with. */
uint32_t vkb_tile_bm(int tile);
uint32_t vkb_tile_bn(int tile);
/* K granularity of one LDS stage for an element type (128 bytes of K). */
uint32_t vkb_tile_bk(int ab_type);

/* Blocked MFMA GEMM for all four layouts.  ab_type F32 -> c_type F32, F16 or BF16;
 * ab_type F16 -> c_type F16 or F32; ab_type BF16 -> c_type BF16 or F32. */
int vkb_launch_gemm(const vkb_gemm_args* a, int tile, void* stream);

/* Split-K pass 2: C = alpha * sum_{s=0}^{split-1} P[s] + beta * C_in + bias,
 * summed in that fixed order (deterministic).  P[s] is M x N fp32, row
 * pitch N, P[s] = P + s*stride_split; epi as vkb_gemm_args.epi. */
int vkb_launch_splitk_reduce(const float* P, int64_t stride_split, uint32_t split,
                             uint32_t M, uint32_t N, void* C, int64_t ldc, int c_type,
                             float alpha, float beta, int scalar_mode,
                             const void* alpha_dev, const void* beta_dev,
                             const vkb_epilogue_args* epi, void* stream);

/* Skinny GEMM for decode (a few activation rows X against a weight W):
 *   C[m][n] = alpha * sum_k X[m][k] * W'[k][n] + beta * C_in[m][n] + bias[n]
 * X = A (K-contiguous rows, lda).  b_kmajor = 1: W = B stored N x K
 * (W'[k][n] = B[n*ldb + k]); b_kmajor = 0: W = B stored K x N
 * (B[k*ldb + n]).  Kernels exist for
 *   fp16 / bf16, b_kmajor, M <= 64, c_type F32 or ab_type;
 *   fp32, either layout, M <= 16, c_type F32 (b_kmajor = 0 needs N % 4 == 0).
 * lda (unless M == 1) and ldb must be multiples of 16 bytes of elements,
 * A and B 16-byte aligned.  vkb_skinny_plan returns the K split the launch
 * must be given (0: no skinny kernel for these arguments); with a split
 * above 1 the kernel writes fp32 partials to part ([split][M][N], row pitch
 * N) and the caller finishes with vkb_launch_splitk_reduce. */
uint32_t vkb_skinny_plan(int ab_type, int b_kmajor, uint32_t M, uint32_t N, uint32_t K, int64_t lda,
                         int64_t ldb);
int vkb_launch_skinny(int ab_type, int b_kmajor, const void* X, int64_t lda, const void* W, int64_t ldb,
                      void* C, int64_t ldc, int c_type,
                      uint32_t M, uint32_t N, uint32_t K,
                      float alpha, float beta, int scalar_mode,
                      const void* alpha_dev, const void* beta_dev,
                      const vkb_epilogue_args* epi,
                      float* part, uint32_t nsplit, void* stream);

#ifdef __cplusplus
}
#endif
