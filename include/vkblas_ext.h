/*
 * vkblas_ext.h — stream-aware entry points of the MI355X-native vkblas.
 *
 * The reference has no counterpart for these: its engine was synchronous and
 * stream-less (src/vkblas.h:27-77) and its hipBLAS shim synchronised the
 * caller's stream before and after every call (src/vkblas_hipblas.c:232).
 * They exist so that the hipBLAS shim can launch on the handle's stream with
 * alpha / beta possibly in device memory, and so that callers with their own
 * stream (tests, benchmarks, PyTorch via ctypes) get the same kernels.
 */
#pragma once
#include "vkblas.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef enum { VKBLAS_DT_F32 = 0, VKBLAS_DT_F16 = 1, VKBLAS_DT_BF16 = 2 } vkblas_dtype_t;

/* Status of the stream-aware entry points (beyond vkblas_status_t): a
 * kernel launch failed after an earlier kernel of the same call had been
 * enqueued to write part of C.  C may then hold results for some rows, so
 * the call must not be repeated by another library on the same C: the
 * hipBLAS, rocBLAS and hipBLASLt entry points report an execution failure
 * for it instead of forwarding the call to the vendor library. */
#define VKBLAS_ERR_PARTIAL ((vkblas_status_t)5)

/* How alpha / beta are passed (hipBLAS pointer modes). */
typedef enum {
    VKBLAS_SCALAR_HOST = 0,     /* the float alpha / beta arguments          */
    VKBLAS_SCALAR_DEV_F32 = 1,  /* alpha_dev / beta_dev point to device f32  */
    VKBLAS_SCALAR_DEV_F16 = 2   /* alpha_dev / beta_dev point to device f16  */
} vkblas_scalar_mode_t;

/* Kernel path chosen for a call (vkblas_last_path, vkblas_plan_gemm). */
typedef enum {
    VKBLAS_PATH_NONE = 0,
    VKBLAS_PATH_TILE64 = 1,   /* blocked MFMA GEMM,  64 x  64 tiles        */
    VKBLAS_PATH_TILE128 = 2,  /* blocked MFMA GEMM, 128 x 128 tiles        */
    VKBLAS_PATH_TILE256 = 3,  /* blocked MFMA GEMM, 256 x 256 tiles        */
    VKBLAS_PATH_SPLITK = 4,   /* split-K pass 1 + deterministic reduce     */
    VKBLAS_PATH_SKINNY = 5,   /* bandwidth-bound decode (M <= 64)          */
    VKBLAS_PATH_TAIL = 6      /* whole waves of tiles, then split-K over
                                 the last tail_rows rows of C             */
} vkblas_path_t;

/* GEMM kernel that ran (vkblas_last_kernel); the values equal the
 * launcher's VKB_KERN_* codes. */
typedef enum {
    VKBLAS_KERNEL_NONE = 0,
    VKBLAS_KERNEL_GENERIC = 1,          /* blocked MFMA kernel, whole tiles        */
    VKBLAS_KERNEL_GENERIC_CHECKED = 2,  /* blocked MFMA kernel with edge handling  */
    VKBLAS_KERNEL_PIPE256 = 3,          /* pipelined kernel, 256 x 256 tiles       */
    VKBLAS_KERNEL_PIPE128 = 4,          /* pipelined kernel, 128 x 128, 2 stages   */
    VKBLAS_KERNEL_PIPE128_4 = 5,        /* pipelined kernel, 128 x 128, 4 stages   */
    VKBLAS_KERNEL_SKINNY = 6,           /* decode kernels                          */
    VKBLAS_KERNEL_WAVEK = 7             /* split-K pass 1 on 32 x 32 / 64 x 64
                                           tiles, the slice's K over the waves  */
} vkblas_kernel_t;

typedef struct {
    int path;              /* vkblas_path_t                                 */
    int tile;              /* tile of the GEMM kernel (0:64, 1:128, 2:256;
                              split-K pass 1 only: 3:32, 4:64 with each K
                              slice divided among four workgroups)         */
    uint32_t split;        /* split-K factor, 1 = no split (VKBLAS_PATH_TAIL:
                              the split of the tail rows)                  */
    uint32_t k_per_split;  /* K per split (multiple of the tile's K step)   */
    uint32_t tail_rows;    /* VKBLAS_PATH_TAIL: rows M - tail_rows .. M - 1
                              run split-K, the rows before them as tiles;
                              0 otherwise                                  */
} vkblas_plan_t;

/*
 * General GEMM on a caller-chosen HIP stream (NULL = null stream).
 *   ab_type: type of A and B; c_type: type of C
 *     (F32, F32) | (F32, F16) | (F32, BF16) | (F16, F16) | (F16, F32) |
 *     (BF16, BF16) | (BF16, F32).
 *     fp32 accumulation throughout; 16-bit results rounded to nearest even.
 *   split_k: 0 = heuristic, 1 = never split, >1 = force that many K slices
 *            (clamped so every slice is non-empty).
 * Returns VKBLAS_OK, VKBLAS_ERR_PARAM (bad arguments / unsupported type
 * combination), VKBLAS_ERR_INIT (no GPU, launch failure before anything
 * was enqueued to write C) or VKBLAS_ERR_PARTIAL (a launch failed after part
 * of C was enqueued to be written: the split tail).  Asynchronous:
 * C is valid once the stream reaches this point.
 */
vkblas_status_t vkblas_gemm_async(
    vkblas_dtype_t ab_type, vkblas_dtype_t c_type,
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    float alpha,
    const void* A, uint32_t lda,
    const void* B, uint32_t ldb,
    float beta,
    void* C, uint32_t ldc,
    uint32_t batch,
    int64_t stride_a, int64_t stride_b, int64_t stride_c,
    vkblas_scalar_mode_t scalar_mode, const void* alpha_dev, const void* beta_dev,
    uint32_t split_k,
    void* stream);

/*
 * Epilogue inputs of vkblas_gemm_ex_async:
 *   C = alpha * op(A) op(B) + beta * C_in + bias[n]
 * computed in fp32 and rounded once to c_type.
 *   c_in:  the matrix beta scales, of c_type, with its own leading dimension
 *          and batch stride; NULL = C itself (the in-place BLAS form).  Read
 *          only when beta != 0.  C_in and C must not overlap unless equal.
 *   bias:  NULL, or N values of bias_type (F32, F16 or BF16): one per column
 *          n of the row-major C, i.e. per row of a column-major (hipBLAS /
 *          hipBLASLt) result, shared by every batch, added after alpha and
 *          beta (hipBLASLt's HIPBLASLT_EPILOGUE_BIAS).
 * No reference counterpart: the reference's engine had neither (PyTorch's
 * addmm bias, reference test/test_torch.py:65-73, reaches the vendor
 * library's bias epilogue on gfx950).
 */
typedef struct {
    const void* c_in;
    uint32_t ldc_in;
    int64_t stride_c_in;
    const void* bias;
    vkblas_dtype_t bias_type;
} vkblas_epilogue_t;

/* vkblas_gemm_async with epilogue inputs (NULL = none: identical to
 * vkblas_gemm_async).  Returns VKBLAS_ERR_PARAM for an unknown bias_type or
 * ldc_in == 0 with c_in set. */
vkblas_status_t vkblas_gemm_ex_async(
    vkblas_dtype_t ab_type, vkblas_dtype_t c_type,
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    float alpha,
    const void* A, uint32_t lda,
    const void* B, uint32_t ldb,
    float beta,
    void* C, uint32_t ldc,
    uint32_t batch,
    int64_t stride_a, int64_t stride_b, int64_t stride_c,
    vkblas_scalar_mode_t scalar_mode, const void* alpha_dev, const void* beta_dev,
    uint32_t split_k,
    const vkblas_epilogue_t* epilogue,
    void* stream);

/*
 * Pointer-array batched GEMM on a HIP stream: A, B, C are device arrays of
 * `batch` matrix pointers (hipblas*gemmBatched), each matrix with the same
 * shape, op and leading dimension; batch b computes
 *   C[b] = alpha * op(A[b]) op(B[b]) + beta * C[b]   (row-major engine contract).
 * Type combinations, scalars and status as vkblas_gemm_async.  The matrices
 * need no particular alignment.  Never split-K or the skinny path (their
 * planning needs the matrix pointers on the host).  No reference counterpart:
 * the reference forwards pointer-array batched calls to the vendor library.
 */
vkblas_status_t vkblas_gemm_batched_async(
    vkblas_dtype_t ab_type, vkblas_dtype_t c_type,
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    float alpha,
    const void* const* A, uint32_t lda,
    const void* const* B, uint32_t ldb,
    float beta,
    void* const* C, uint32_t ldc,
    uint32_t batch,
    vkblas_scalar_mode_t scalar_mode, const void* alpha_dev, const void* beta_dev,
    void* stream);

/* The path planned for a call with these arguments (no GPU needed).
 * aligned: A, B, C base pointers 16-byte aligned (the skinny kernel needs it).
 * Returns VKBLAS_OK or VKBLAS_ERR_PARAM. */
vkblas_status_t vkblas_plan_gemm(
    vkblas_dtype_t ab_type, vkblas_dtype_t c_type,
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    uint32_t lda, uint32_t ldb, uint32_t ldc,
    uint32_t batch, uint32_t split_k, int aligned,
    vkblas_plan_t* plan);

/* Process-wide kernel override for testing and tuning (the VKBLAS_TILE /
 * VKBLAS_KERNEL environment variables set the same at load time).
 *   tile:    -1 = planner's choice, 0 = 64x64, 1 = 128x128, 2 = 256x256
 *   generic: 1 = always the generic blocked kernel (no pipelined variant)
 * Returns VKBLAS_ERR_PARAM for an unknown tile. */
vkblas_status_t vkblas_set_override(int tile, int generic);

/* Path taken by the calling thread's most recent successful GEMM call. */
int vkblas_last_path(void);

/* Kernel (vkblas_kernel_t) the calling thread's most recent successful GEMM
 * call launched (split-K: its pass-1 kernel). */
int vkblas_last_kernel(void);

/*
 * vkblas_gemm_async that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, plan, kernels and results as
 * vkblas_gemm_async; the split-K and split-decode partials ([split][M][N]
 * fp32) go to a fixed per-device scratch array of
 * vkblas_noalloc_scratch_bytes() (64 MiB of partials after 4 KiB of split-K
 * arrival counters) instead of an allocated workspace.  A call whose
 * partials need more returns VKBLAS_ERR_PARAM before launching anything
 * (e.g. split_k = 128 on a 1024 x 1024 output).
 * All calls on one device share its array: calls that overlap in time on
 * one device (other streams, unordered threads) race and must be ordered by
 * the caller.
 */
vkblas_status_t vkblas_gemm_noalloc_async(
    vkblas_dtype_t ab_type, vkblas_dtype_t c_type,
    vkblas_op_t op_a, vkblas_op_t op_b,
    uint32_t M, uint32_t N, uint32_t K,
    float alpha,
    const void* A, uint32_t lda,
    const void* B, uint32_t ldb,
    float beta,
    void* C, uint32_t ldc,
    uint32_t batch,
    int64_t stride_a, int64_t stride_b, int64_t stride_c,
    vkblas_scalar_mode_t scalar_mode, const void* alpha_dev, const void* beta_dev,
    uint32_t split_k,
    void* stream);

/* Size in bytes of the per-device scratch array of vkblas_gemm_noalloc_async. */
size_t vkblas_noalloc_scratch_bytes(void);

/* Frees the split-K / decode partial buffers the library keeps per stream
 * between calls (they are otherwise kept until the process ends, at most
 * 4 GiB in all).  Waits for all work on every device that holds one.  Call
 * it while no other thread is inside the library; later calls allocate
 * again.  Returns VKBLAS_OK, or VKBLAS_ERR_INIT if a HIP call failed.  No
 * reference counterpart (the reference's partials were grow-only,
 * src/vkblas.c:1889-1914). */
vkblas_status_t vkblas_workspace_release(void);

/* Library version string. */
const char* vkblas_version(void);

#ifdef __cplusplus
}
#endif
