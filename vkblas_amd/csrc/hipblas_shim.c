/*
 * hipblas_shim.c — hipBLAS ABI entry points of libvkblas_hipblas.so (C11).
 *
 * Drop-in for the reference's LD_PRELOAD shim (src/vkblas_hipblas.c).  The
 * fp32 / fp16 / bf16 GEMM family is computed by this library's gfx950 kernels; every
 * other exported hipBLAS symbol, and every GEMM call this library declines,
 * is forwarded to the real hipBLAS of the process.
 *
 * Column-major -> row-major translation (reference src/vkblas_hipblas.c:187-189,
 * 234-239): hipBLAS C(m x n) = op(A) op(B), column-major, is the row-major
 * C'(n x m) = op(B)' op(A)', so the engine runs with
 *     op_a = transB, op_b = transA, M = n, N = m, A = B, lda = ldb, B = A, ldb = lda.
 *
 * Differences from the reference, on purpose:
 *   - stream and pointer mode are read from the handle (per-handle state held
 *     by the real hipBLAS) instead of process globals (reference lines 46-47);
 *   - launches are asynchronous on the handle's stream; no host sync before
 *     or after (reference line 232);
 *   - HIPBLAS_POINTER_MODE_DEVICE scalars are read by the kernels, not copied
 *     to the host (reference get_scalar_f32, lines 126-131);
 *   - fp16 inputs with fp32 output (GemmEx 16F/16F/32F), hipblasHgemm* and the
 *     unsuffixed GemmStridedBatchedEx are intercepted too;
 *   - m, n, k or batchCount <= 0, invalid leading dimensions, and sizes beyond
 *     32 bits are forwarded to the real hipBLAS so its quick-return and error
 *     semantics apply unchanged (the reference returned INVALID_VALUE for
 *     m, n, k <= 0, reference line 223);
 *   - hipFree / hipHostFree / hipFreeManaged are NOT interposed: there is no
 *     import cache to invalidate (reference lines 160-184).
 */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <hip/hip_runtime_api.h>
#include <hipblas/hipblas.h>

#include "vkblas_ext.h"
#include "vkblas_hipblas.h"

/* ------------------------------------------------------ real hipBLAS lookup */

static pthread_once_t g_real_once = PTHREAD_ONCE_INIT;
static void* g_real = NULL;
static void* g_self_base = NULL;
static int g_trace = 0;

static void self_anchor(void) {}

static int in_self(void* f) {
    Dl_info info;
    if (!f) return 0;
    if (!dladdr(f, &info)) return 0;
    return info.dli_fbase == g_self_base;
}

static void real_open(void) {
    Dl_info info;
    const char* e = getenv("VKBLAS_TRACE");
    g_trace = e && e[0] && e[0] != '0';
    if (dladdr((void*)&self_anchor, &info)) g_self_base = info.dli_fbase;
    static const char* names[] = {"libhipblas.so.3", "libhipblas.so", "libhipblas.so.2",
                                  "/opt/rocm/lib/libhipblas.so.3"};
    const int n = (int)(sizeof(names) / sizeof(names[0]));
    /* prefer the instance the process already uses */
    for (int i = 0; i < n && !g_real; ++i) {
        void* h = dlopen(names[i], RTLD_LAZY | RTLD_NOLOAD);
        if (h) {
            void* probe = dlsym(h, "hipblasCreate");
            if (probe && !in_self(probe)) g_real = h;
            else dlclose(h);
        }
    }
    for (int i = 0; i < n && !g_real; ++i) {
        void* h = dlopen(names[i], RTLD_LAZY | RTLD_LOCAL);
        if (h) {
            void* probe = dlsym(h, "hipblasCreate");
            if (probe && !in_self(probe)) g_real = h;
            else dlclose(h);
        }
    }
    if (!g_real && g_trace) fprintf(stderr, "[vkblas] real libhipblas not found: forwarding disabled\n");
}

/* Resolve a symbol of the real hipBLAS; never returns one of our own. */
static void* real_sym(const char* name) {
    pthread_once(&g_real_once, real_open);
    void* f = dlsym(RTLD_NEXT, name);
    if (f && !in_self(f)) return f;
    if (g_real) {
        f = dlsym(g_real, name);
        if (f && !in_self(f)) return f;
    }
    return NULL;
}

/* Forwarder: exports `name` with parameter list `params`, calls the real
 * symbol `real_name` with `args`, or returns `err` if it cannot be found. */
#define VKB_FWD(ret_t, err, name, real_name, params, args)                      \
    ret_t name params {                                                         \
        static void* fn_;                                                       \
        void* f_ = __atomic_load_n(&fn_, __ATOMIC_ACQUIRE);                     \
        if (!f_) {                                                              \
            f_ = real_sym(#real_name);                                          \
            __atomic_store_n(&fn_, f_, __ATOMIC_RELEASE);                       \
        }                                                                       \
        return f_ ? ((ret_t(*) params)f_) args : (err);                         \
    }

#define NS HIPBLAS_STATUS_NOT_SUPPORTED

/* ------------------------------------------------ handle and state (forward) */

/* hipblasCreate returns the real handle: callers (PyTorch) use it with the
 * real library directly (reference src/vkblas_hipblas.c:43-45, 69-75). */
VKB_FWD(hipblasStatus_t, NS, hipblasCreate, hipblasCreate, (hipblasHandle_t* handle), (handle))
VKB_FWD(hipblasStatus_t, NS, hipblasDestroy, hipblasDestroy, (hipblasHandle_t handle), (handle))
VKB_FWD(hipblasStatus_t, NS, hipblasSetStream, hipblasSetStream, (hipblasHandle_t handle, hipStream_t s),
        (handle, s))
VKB_FWD(hipblasStatus_t, NS, hipblasGetStream, hipblasGetStream, (hipblasHandle_t handle, hipStream_t* s),
        (handle, s))
VKB_FWD(hipblasStatus_t, NS, hipblasSetPointerMode, hipblasSetPointerMode,
        (hipblasHandle_t handle, hipblasPointerMode_t mode), (handle, mode))
VKB_FWD(hipblasStatus_t, NS, hipblasGetPointerMode, hipblasGetPointerMode,
        (hipblasHandle_t handle, hipblasPointerMode_t* mode), (handle, mode))
VKB_FWD(hipblasStatus_t, NS, hipblasSetAtomicsMode, hipblasSetAtomicsMode,
        (hipblasHandle_t handle, hipblasAtomicsMode_t mode), (handle, mode))

hipblasStatus_t hipblasGetVersion(hipblasHandle_t handle, int* version);
VKB_FWD(hipblasStatus_t, NS, hipblasGetVersion, hipblasGetVersion, (hipblasHandle_t handle, int* version),
        (handle, version))

/* Workspace only matters to the vendor library; a handle whose real
 * library lacks the call still reports success, as the reference did
 * (src/vkblas_hipblas.c:105-112) so PyTorch's status check passes. */
hipblasStatus_t hipblasSetWorkspace(hipblasHandle_t handle, void* workspace, size_t size) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    typedef hipblasStatus_t (*fn_t)(hipblasHandle_t, void*, size_t);
    fn_t f = (fn_t)real_sym("hipblasSetWorkspace");
    return f ? f(handle, workspace, size) : HIPBLAS_STATUS_SUCCESS;
}

const char* hipblasStatusToString(hipblasStatus_t status) {
    typedef const char* (*fn_t)(hipblasStatus_t);
    fn_t f = (fn_t)real_sym("hipblasStatusToString");
    return f ? f(status) : "unknown";
}

/* ------------------------------------------------------------ GEMM family */

#define VKB_DECLINE ((hipblasStatus_t)-1)

static float half_bits_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else {
            int e = -1;
            do { man <<= 1; ++e; } while (!(man & 0x400u));
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static int op_is_t(hipblasOperation_t op) { return op == HIPBLAS_OP_T || op == HIPBLAS_OP_C; }

/* Runs the GEMM on this library's kernels, or returns VKB_DECLINE for the
 * caller to forward.  ab / ct: element types; scal_f16: alpha and beta are
 * hipblasHalf (else float). */
static const char* dtype_name(vkblas_dtype_t t) {
    return t == VKBLAS_DT_F16 ? "f16" : t == VKBLAS_DT_BF16 ? "bf16" : "f32";
}

/* ptr_array: A, B, C are device arrays of batch matrix pointers
 * (hipblas*gemmBatched); the strides are then unused. */
static hipblasStatus_t run_gemm_any(hipblasHandle_t handle, vkblas_dtype_t ab, vkblas_dtype_t ct, int scal_f16,
                                    hipblasOperation_t transA, hipblasOperation_t transB,
                                    int64_t m, int64_t n, int64_t k, const void* alpha,
                                    const void* A, int64_t lda, int64_t sA,
                                    const void* B, int64_t ldb, int64_t sB, const void* beta,
                                    void* C, int64_t ldc, int64_t sC, int64_t batch, int ptr_array) {
    pthread_once(&g_real_once, real_open);
    if (m <= 0 || n <= 0 || k <= 0 || batch <= 0) return VKB_DECLINE;
    if (m > UINT32_MAX || n > UINT32_MAX || k > UINT32_MAX || batch > UINT32_MAX) return VKB_DECLINE;
    if (lda > UINT32_MAX || ldb > UINT32_MAX || ldc > UINT32_MAX) return VKB_DECLINE;
    /* hipBLAS argument rules: the real library reports violations */
    if (lda < (op_is_t(transA) ? k : m) || ldb < (op_is_t(transB) ? n : k) || ldc < m) return VKB_DECLINE;
    if (!alpha || !beta) return VKB_DECLINE;

    hipStream_t stream = NULL;
    hipblasPointerMode_t mode = HIPBLAS_POINTER_MODE_HOST;
    {
        typedef hipblasStatus_t (*gs_t)(hipblasHandle_t, hipStream_t*);
        typedef hipblasStatus_t (*gm_t)(hipblasHandle_t, hipblasPointerMode_t*);
        static void* gs_fn;
        static void* gm_fn;
        void* gs = __atomic_load_n(&gs_fn, __ATOMIC_ACQUIRE);
        void* gm = __atomic_load_n(&gm_fn, __ATOMIC_ACQUIRE);
        if (!gs) { gs = real_sym("hipblasGetStream"); __atomic_store_n(&gs_fn, gs, __ATOMIC_RELEASE); }
        if (!gm) { gm = real_sym("hipblasGetPointerMode"); __atomic_store_n(&gm_fn, gm, __ATOMIC_RELEASE); }
        if (gs && ((gs_t)gs)(handle, &stream) != HIPBLAS_STATUS_SUCCESS) return VKB_DECLINE;
        if (gm && ((gm_t)gm)(handle, &mode) != HIPBLAS_STATUS_SUCCESS) return VKB_DECLINE;
    }

    float a = 0.0f, b = 0.0f;
    vkblas_scalar_mode_t sm = VKBLAS_SCALAR_HOST;
    const void* ad = NULL;
    const void* bd = NULL;
    if (mode == HIPBLAS_POINTER_MODE_DEVICE) {
        sm = scal_f16 ? VKBLAS_SCALAR_DEV_F16 : VKBLAS_SCALAR_DEV_F32;
        ad = alpha;
        bd = beta;
    } else if (scal_f16) {
        a = half_bits_to_float(*(const uint16_t*)alpha);
        b = half_bits_to_float(*(const uint16_t*)beta);
    } else {
        a = *(const float*)alpha;
        b = *(const float*)beta;
    }
    if (g_trace)
        fprintf(stderr, "[vkblas] hipblas gemm%s %s%s %s->%s m=%lld n=%lld k=%lld lda=%lld ldb=%lld ldc=%lld "
                        "batch=%lld\n",
                ptr_array ? " batched" : "", op_is_t(transA) ? "T" : "N", op_is_t(transB) ? "T" : "N",
                dtype_name(ab), dtype_name(ct), (long long)m, (long long)n, (long long)k, (long long)lda,
                (long long)ldb, (long long)ldc, (long long)batch);
    const vkblas_op_t op_a = op_is_t(transB) ? VKBLAS_OP_T : VKBLAS_OP_N;
    const vkblas_op_t op_b = op_is_t(transA) ? VKBLAS_OP_T : VKBLAS_OP_N;
    vkblas_status_t st;
    if (ptr_array)
        st = vkblas_gemm_batched_async(ab, ct, op_a, op_b, (uint32_t)n, (uint32_t)m, (uint32_t)k, a,
                                       (const void* const*)B, (uint32_t)ldb, (const void* const*)A, (uint32_t)lda,
                                       b, (void* const*)C, (uint32_t)ldc, (uint32_t)batch, sm, ad, bd, stream);
    else
        st = vkblas_gemm_async(ab, ct, op_a, op_b, (uint32_t)n, (uint32_t)m, (uint32_t)k, a, B, (uint32_t)ldb, A,
                               (uint32_t)lda, b, C, (uint32_t)ldc, (uint32_t)batch, batch > 1 ? sB : 0,
                               batch > 1 ? sA : 0, batch > 1 ? sC : 0, sm, ad, bd, 0, stream);
    if (st == VKBLAS_ERR_PARTIAL) {
        /* part of C may already be written: repeating the call elsewhere
         * could read it as its input C */
        if (g_trace) fprintf(stderr, "[vkblas] engine status %d: execution failed, not forwarded\n", (int)st);
        return HIPBLAS_STATUS_EXECUTION_FAILED;
    }
    if (st != VKBLAS_OK) {
        if (g_trace) fprintf(stderr, "[vkblas] engine status %d: forwarding\n", (int)st);
        return VKB_DECLINE;
    }
    return HIPBLAS_STATUS_SUCCESS;
}

static hipblasStatus_t run_gemm(hipblasHandle_t handle, vkblas_dtype_t ab, vkblas_dtype_t ct, int scal_f16,
                                hipblasOperation_t transA, hipblasOperation_t transB,
                                int64_t m, int64_t n, int64_t k, const void* alpha,
                                const void* A, int64_t lda, int64_t sA,
                                const void* B, int64_t ldb, int64_t sB, const void* beta,
                                void* C, int64_t ldc, int64_t sC, int64_t batch) {
    return run_gemm_any(handle, ab, ct, scal_f16, transA, transB, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C,
                        ldc, sC, batch, 0);
}

static hipblasStatus_t run_gemm_batched(hipblasHandle_t handle, vkblas_dtype_t ab, vkblas_dtype_t ct, int scal_f16,
                                        hipblasOperation_t transA, hipblasOperation_t transB,
                                        int64_t m, int64_t n, int64_t k, const void* alpha,
                                        const void* A, int64_t lda, const void* B, int64_t ldb, const void* beta,
                                        void* C, int64_t ldc, int64_t batch) {
    return run_gemm_any(handle, ab, ct, scal_f16, transA, transB, m, n, k, alpha, A, lda, 0, B, ldb, 0, beta, C,
                        ldc, 0, batch, 1);
}

/* Data / compute type classification.  Values of the pre-3.0
 * hipblasDatatype_t (150 = R_16F, 151 = R_32F, 168 = R_16B) are accepted as
 * well, as the reference did (src/vkblas_hipblas.c:280-284). */
static int is_f32_t(int t) { return t == HIP_R_32F || t == 151; }
static int is_f16_t(int t) { return t == HIP_R_16F || t == 150; }
static int is_bf16_t(int t) { return t == HIP_R_16BF || t == 168; }
/* 1: float scalars, fp32 accumulate; 2: half scalars (COMPUTE_16F);
 * 0: not handled here.  Full-precision fp32 arithmetic is always an allowed
 * implementation of the FAST_* compute types. */
static int compute_kind(int c) {
    switch (c) {
        case HIPBLAS_COMPUTE_32F:
        case HIPBLAS_COMPUTE_32F_PEDANTIC:
        case HIPBLAS_COMPUTE_32F_FAST_16F:
        case HIPBLAS_COMPUTE_32F_FAST_16BF:
        case HIPBLAS_COMPUTE_32F_FAST_TF32:
        case 151:
            return 1;
        case HIPBLAS_COMPUTE_16F:
        case 150:
            return 2;
        default:
            return 0;
    }
}

/* Classify a GemmEx type combination: returns 1 and sets ab/ct/scal_f16 when
 * this library computes it. */
static int ex_types(int at, int bt, int ctp, int comp, vkblas_dtype_t* ab, vkblas_dtype_t* ct, int* scal_f16) {
    const int kind = compute_kind(comp);
    if (kind == 0) return 0;
    if (is_f32_t(at) && is_f32_t(bt) && kind == 1 && (is_f32_t(ctp) || is_f16_t(ctp) || is_bf16_t(ctp))) {
        /* fp32 in, fp32 / fp16 / bf16 out (the 16-bit results rounded once) */
        *ab = VKBLAS_DT_F32;
        *ct = is_f32_t(ctp) ? VKBLAS_DT_F32 : is_f16_t(ctp) ? VKBLAS_DT_F16 : VKBLAS_DT_BF16;
        *scal_f16 = 0;
        return 1;
    }
    if (is_f16_t(at) && is_f16_t(bt) && (is_f16_t(ctp) || is_f32_t(ctp))) {
        if (kind == 2 && !is_f16_t(ctp)) return 0;
        *ab = VKBLAS_DT_F16;
        *ct = is_f16_t(ctp) ? VKBLAS_DT_F16 : VKBLAS_DT_F32;
        *scal_f16 = kind == 2;
        return 1;
    }
    /* bf16 (reference src/vkblas_hipblas.c:426-461 routes 16BF -> 16BF; a
     * 32F result is computed here too).  hipBLAS defines bf16 GEMMs with fp32
     * compute only, so alpha / beta are floats. */
    if (is_bf16_t(at) && is_bf16_t(bt) && (is_bf16_t(ctp) || is_f32_t(ctp)) && kind == 1) {
        *ab = VKBLAS_DT_BF16;
        *ct = is_bf16_t(ctp) ? VKBLAS_DT_BF16 : VKBLAS_DT_F32;
        *scal_f16 = 0;
        return 1;
    }
    return 0;
}

#define REAL_CALL(ret_t, real_name, params, args)                               \
    do {                                                                        \
        static void* fn_;                                                       \
        void* f_ = __atomic_load_n(&fn_, __ATOMIC_ACQUIRE);                     \
        if (!f_) {                                                              \
            f_ = real_sym(#real_name);                                          \
            __atomic_store_n(&fn_, f_, __ATOMIC_RELEASE);                       \
        }                                                                       \
        return f_ ? ((ret_t(*) params)f_) args : NS;                            \
    } while (0)

/* reference src/vkblas_hipblas.c:403-408 */
hipblasStatus_t hipblasSgemm(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                             int m, int n, int k, const float* alpha, const float* AP, int lda,
                             const float* BP, int ldb, const float* beta, float* CP, int ldc) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm(handle, VKBLAS_DT_F32, VKBLAS_DT_F32, 0, transA, transB, m, n, k, alpha, AP,
                                 lda, 0, BP, ldb, 0, beta, CP, ldc, 0, 1);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasSgemm,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int, int, int, const float*,
               const float*, int, const float*, int, const float*, float*, int),
              (handle, transA, transB, m, n, k, alpha, AP, lda, BP, ldb, beta, CP, ldc));
}

hipblasStatus_t hipblasSgemm_64(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                int64_t m, int64_t n, int64_t k, const float* alpha, const float* AP,
                                int64_t lda, const float* BP, int64_t ldb, const float* beta, float* CP,
                                int64_t ldc) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm(handle, VKBLAS_DT_F32, VKBLAS_DT_F32, 0, transA, transB, m, n, k, alpha, AP,
                                 lda, 0, BP, ldb, 0, beta, CP, ldc, 0, 1);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasSgemm_64,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int64_t, int64_t, int64_t,
               const float*, const float*, int64_t, const float*, int64_t, const float*, float*, int64_t),
              (handle, transA, transB, m, n, k, alpha, AP, lda, BP, ldb, beta, CP, ldc));
}

/* reference src/vkblas_hipblas.c:409-416 */
hipblasStatus_t hipblasSgemmStridedBatched(hipblasHandle_t handle, hipblasOperation_t transA,
                                           hipblasOperation_t transB, int m, int n, int k, const float* alpha,
                                           const float* AP, int lda, long long strideA, const float* BP,
                                           int ldb, long long strideB, const float* beta, float* CP, int ldc,
                                           long long strideC, int batchCount) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm(handle, VKBLAS_DT_F32, VKBLAS_DT_F32, 0, transA, transB, m, n, k, alpha, AP,
                                 lda, strideA, BP, ldb, strideB, beta, CP, ldc, strideC, batchCount);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasSgemmStridedBatched,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int, int, int, const float*,
               const float*, int, long long, const float*, int, long long, const float*, float*, int,
               long long, int),
              (handle, transA, transB, m, n, k, alpha, AP, lda, strideA, BP, ldb, strideB, beta, CP, ldc,
               strideC, batchCount));
}

hipblasStatus_t hipblasSgemmStridedBatched_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                              hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                              const float* alpha, const float* AP, int64_t lda,
                                              long long strideA, const float* BP, int64_t ldb,
                                              long long strideB, const float* beta, float* CP, int64_t ldc,
                                              long long strideC, int64_t batchCount) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm(handle, VKBLAS_DT_F32, VKBLAS_DT_F32, 0, transA, transB, m, n, k, alpha, AP,
                                 lda, strideA, BP, ldb, strideB, beta, CP, ldc, strideC, batchCount);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasSgemmStridedBatched_64,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int64_t, int64_t, int64_t,
               const float*, const float*, int64_t, long long, const float*, int64_t, long long,
               const float*, float*, int64_t, long long, int64_t),
              (handle, transA, transB, m, n, k, alpha, AP, lda, strideA, BP, ldb, strideB, beta, CP, ldc,
               strideC, batchCount));
}

/* fp16 with hipblasHalf alpha/beta; new relative to the reference */
hipblasStatus_t hipblasHgemm(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                             int m, int n, int k, const hipblasHalf* alpha, const hipblasHalf* AP, int lda,
                             const hipblasHalf* BP, int ldb, const hipblasHalf* beta, hipblasHalf* CP,
                             int ldc) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm(handle, VKBLAS_DT_F16, VKBLAS_DT_F16, 1, transA, transB, m, n, k, alpha, AP,
                                 lda, 0, BP, ldb, 0, beta, CP, ldc, 0, 1);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasHgemm,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int, int, int, const hipblasHalf*,
               const hipblasHalf*, int, const hipblasHalf*, int, const hipblasHalf*, hipblasHalf*, int),
              (handle, transA, transB, m, n, k, alpha, AP, lda, BP, ldb, beta, CP, ldc));
}

hipblasStatus_t hipblasHgemm_64(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                int64_t m, int64_t n, int64_t k, const hipblasHalf* alpha,
                                const hipblasHalf* AP, int64_t lda, const hipblasHalf* BP, int64_t ldb,
                                const hipblasHalf* beta, hipblasHalf* CP, int64_t ldc) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm(handle, VKBLAS_DT_F16, VKBLAS_DT_F16, 1, transA, transB, m, n, k, alpha, AP,
                                 lda, 0, BP, ldb, 0, beta, CP, ldc, 0, 1);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasHgemm_64,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int64_t, int64_t, int64_t,
               const hipblasHalf*, const hipblasHalf*, int64_t, const hipblasHalf*, int64_t,
               const hipblasHalf*, hipblasHalf*, int64_t),
              (handle, transA, transB, m, n, k, alpha, AP, lda, BP, ldb, beta, CP, ldc));
}

hipblasStatus_t hipblasHgemmStridedBatched(hipblasHandle_t handle, hipblasOperation_t transA,
                                           hipblasOperation_t transB, int m, int n, int k,
                                           const hipblasHalf* alpha, const hipblasHalf* AP, int lda,
                                           long long strideA, const hipblasHalf* BP, int ldb, long long strideB,
                                           const hipblasHalf* beta, hipblasHalf* CP, int ldc, long long strideC,
                                           int batchCount) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm(handle, VKBLAS_DT_F16, VKBLAS_DT_F16, 1, transA, transB, m, n, k, alpha, AP,
                                 lda, strideA, BP, ldb, strideB, beta, CP, ldc, strideC, batchCount);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasHgemmStridedBatched,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int, int, int, const hipblasHalf*,
               const hipblasHalf*, int, long long, const hipblasHalf*, int, long long, const hipblasHalf*,
               hipblasHalf*, int, long long, int),
              (handle, transA, transB, m, n, k, alpha, AP, lda, strideA, BP, ldb, strideB, beta, CP, ldc,
               strideC, batchCount));
}

hipblasStatus_t hipblasHgemmStridedBatched_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                              hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                              const hipblasHalf* alpha, const hipblasHalf* AP, int64_t lda,
                                              long long strideA, const hipblasHalf* BP, int64_t ldb,
                                              long long strideB, const hipblasHalf* beta, hipblasHalf* CP,
                                              int64_t ldc, long long strideC, int64_t batchCount) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm(handle, VKBLAS_DT_F16, VKBLAS_DT_F16, 1, transA, transB, m, n, k, alpha, AP,
                                 lda, strideA, BP, ldb, strideB, beta, CP, ldc, strideC, batchCount);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasHgemmStridedBatched_64,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int64_t, int64_t, int64_t,
               const hipblasHalf*, const hipblasHalf*, int64_t, long long, const hipblasHalf*, int64_t,
               long long, const hipblasHalf*, hipblasHalf*, int64_t, long long, int64_t),
              (handle, transA, transB, m, n, k, alpha, AP, lda, strideA, BP, ldb, strideB, beta, CP, ldc,
               strideC, batchCount));
}

/* reference src/vkblas_hipblas.c:454-466 (hipBLAS >= 3 signature, lines 19-35) */
hipblasStatus_t hipblasGemmEx(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                              int m, int n, int k, const void* alpha, const void* A, hipDataType aType, int lda,
                              const void* B, hipDataType bType, int ldb, const void* beta, void* C,
                              hipDataType cType, int ldc, hipblasComputeType_t computeType,
                              hipblasGemmAlgo_t algo) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    vkblas_dtype_t ab, ct;
    int sf16;
    if (ex_types((int)aType, (int)bType, (int)cType, (int)computeType, &ab, &ct, &sf16)) {
        hipblasStatus_t s = run_gemm(handle, ab, ct, sf16, transA, transB, m, n, k, alpha, A, lda, 0, B, ldb,
                                     0, beta, C, ldc, 0, 1);
        if (s != VKB_DECLINE) return s;
    }
    REAL_CALL(hipblasStatus_t, hipblasGemmEx,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int, int, int, const void*, const void*,
               hipDataType, int, const void*, hipDataType, int, const void*, void*, hipDataType, int,
               hipblasComputeType_t, hipblasGemmAlgo_t),
              (handle, transA, transB, m, n, k, alpha, A, aType, lda, B, bType, ldb, beta, C, cType, ldc,
               computeType, algo));
}

/* reference src/vkblas_hipblas.c:417-432.  hipBLAS 3 dropped the _v2 names;
 * the signature is the unsuffixed one, which the real library still has. */
hipblasStatus_t hipblasGemmEx_v2(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                 int m, int n, int k, const void* alpha, const void* A, hipDataType aType,
                                 int lda, const void* B, hipDataType bType, int ldb, const void* beta, void* C,
                                 hipDataType cType, int ldc, hipblasComputeType_t computeType,
                                 hipblasGemmAlgo_t algo) {
    return hipblasGemmEx(handle, transA, transB, m, n, k, alpha, A, aType, lda, B, bType, ldb, beta, C, cType,
                         ldc, computeType, algo);
}

hipblasStatus_t hipblasGemmEx_64(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                 int64_t m, int64_t n, int64_t k, const void* alpha, const void* A,
                                 hipDataType aType, int64_t lda, const void* B, hipDataType bType, int64_t ldb,
                                 const void* beta, void* C, hipDataType cType, int64_t ldc,
                                 hipblasComputeType_t computeType, hipblasGemmAlgo_t algo) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    vkblas_dtype_t ab, ct;
    int sf16;
    if (ex_types((int)aType, (int)bType, (int)cType, (int)computeType, &ab, &ct, &sf16)) {
        hipblasStatus_t s = run_gemm(handle, ab, ct, sf16, transA, transB, m, n, k, alpha, A, lda, 0, B, ldb,
                                     0, beta, C, ldc, 0, 1);
        if (s != VKB_DECLINE) return s;
    }
    REAL_CALL(hipblasStatus_t, hipblasGemmEx_64,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int64_t, int64_t, int64_t, const void*,
               const void*, hipDataType, int64_t, const void*, hipDataType, int64_t, const void*, void*,
               hipDataType, int64_t, hipblasComputeType_t, hipblasGemmAlgo_t),
              (handle, transA, transB, m, n, k, alpha, A, aType, lda, B, bType, ldb, beta, C, cType, ldc,
               computeType, algo));
}

hipblasStatus_t hipblasGemmStridedBatchedEx(hipblasHandle_t handle, hipblasOperation_t transA,
                                            hipblasOperation_t transB, int m, int n, int k, const void* alpha,
                                            const void* A, hipDataType aType, int lda, hipblasStride strideA,
                                            const void* B, hipDataType bType, int ldb, hipblasStride strideB,
                                            const void* beta, void* C, hipDataType cType, int ldc,
                                            hipblasStride strideC, int batchCount,
                                            hipblasComputeType_t computeType, hipblasGemmAlgo_t algo) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    vkblas_dtype_t ab, ct;
    int sf16;
    if (ex_types((int)aType, (int)bType, (int)cType, (int)computeType, &ab, &ct, &sf16)) {
        hipblasStatus_t s = run_gemm(handle, ab, ct, sf16, transA, transB, m, n, k, alpha, A, lda, strideA, B,
                                     ldb, strideB, beta, C, ldc, strideC, batchCount);
        if (s != VKB_DECLINE) return s;
    }
    REAL_CALL(hipblasStatus_t, hipblasGemmStridedBatchedEx,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int, int, int, const void*, const void*,
               hipDataType, int, hipblasStride, const void*, hipDataType, int, hipblasStride, const void*,
               void*, hipDataType, int, hipblasStride, int, hipblasComputeType_t, hipblasGemmAlgo_t),
              (handle, transA, transB, m, n, k, alpha, A, aType, lda, strideA, B, bType, ldb, strideB, beta, C,
               cType, ldc, strideC, batchCount, computeType, algo));
}

/* reference src/vkblas_hipblas.c:433-453 */
hipblasStatus_t hipblasGemmStridedBatchedEx_v2(hipblasHandle_t handle, hipblasOperation_t transA,
                                               hipblasOperation_t transB, int m, int n, int k,
                                               const void* alpha, const void* A, hipDataType aType, int lda,
                                               hipblasStride strideA, const void* B, hipDataType bType,
                                               int ldb, hipblasStride strideB, const void* beta, void* C,
                                               hipDataType cType, int ldc, hipblasStride strideC,
                                               int batchCount, hipblasComputeType_t computeType,
                                               hipblasGemmAlgo_t algo) {
    return hipblasGemmStridedBatchedEx(handle, transA, transB, m, n, k, alpha, A, aType, lda, strideA, B,
                                       bType, ldb, strideB, beta, C, cType, ldc, strideC, batchCount,
                                       computeType, algo);
}

hipblasStatus_t hipblasGemmStridedBatchedEx_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                               hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                               const void* alpha, const void* A, hipDataType aType,
                                               int64_t lda, hipblasStride strideA, const void* B,
                                               hipDataType bType, int64_t ldb, hipblasStride strideB,
                                               const void* beta, void* C, hipDataType cType, int64_t ldc,
                                               hipblasStride strideC, int64_t batchCount,
                                               hipblasComputeType_t computeType, hipblasGemmAlgo_t algo) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    vkblas_dtype_t ab, ct;
    int sf16;
    if (ex_types((int)aType, (int)bType, (int)cType, (int)computeType, &ab, &ct, &sf16)) {
        hipblasStatus_t s = run_gemm(handle, ab, ct, sf16, transA, transB, m, n, k, alpha, A, lda, strideA, B,
                                     ldb, strideB, beta, C, ldc, strideC, batchCount);
        if (s != VKB_DECLINE) return s;
    }
    REAL_CALL(hipblasStatus_t, hipblasGemmStridedBatchedEx_64,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int64_t, int64_t, int64_t, const void*,
               const void*, hipDataType, int64_t, hipblasStride, const void*, hipDataType, int64_t,
               hipblasStride, const void*, void*, hipDataType, int64_t, hipblasStride, int64_t,
               hipblasComputeType_t, hipblasGemmAlgo_t),
              (handle, transA, transB, m, n, k, alpha, A, aType, lda, strideA, B, bType, ldb, strideB, beta, C,
               cType, ldc, strideC, batchCount, computeType, algo));
}

/* -------------------------------------------- pointer-array batched */
/* No reference counterpart: the reference left these to the real hipBLAS.
 * A, B, C are device arrays of batchCount matrix pointers. */

hipblasStatus_t hipblasSgemmBatched(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                    int m, int n, int k, const float* alpha, const float* const AP[], int lda,
                                    const float* const BP[], int ldb, const float* beta, float* const CP[], int ldc,
                                    int batchCount) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm_batched(handle, VKBLAS_DT_F32, VKBLAS_DT_F32, 0, transA, transB, m, n, k, alpha,
                                         AP, lda, BP, ldb, beta, (void*)CP, ldc, batchCount);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasSgemmBatched,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int, int, int, const float*,
               const float* const*, int, const float* const*, int, const float*, float* const*, int, int),
              (handle, transA, transB, m, n, k, alpha, AP, lda, BP, ldb, beta, CP, ldc, batchCount));
}

hipblasStatus_t hipblasSgemmBatched_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                       hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                       const float* alpha, const float* const AP[], int64_t lda,
                                       const float* const BP[], int64_t ldb, const float* beta, float* const CP[],
                                       int64_t ldc, int64_t batchCount) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm_batched(handle, VKBLAS_DT_F32, VKBLAS_DT_F32, 0, transA, transB, m, n, k, alpha,
                                         AP, lda, BP, ldb, beta, (void*)CP, ldc, batchCount);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasSgemmBatched_64,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int64_t, int64_t, int64_t, const float*,
               const float* const*, int64_t, const float* const*, int64_t, const float*, float* const*, int64_t,
               int64_t),
              (handle, transA, transB, m, n, k, alpha, AP, lda, BP, ldb, beta, CP, ldc, batchCount));
}

hipblasStatus_t hipblasHgemmBatched(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                    int m, int n, int k, const hipblasHalf* alpha, const hipblasHalf* const AP[],
                                    int lda, const hipblasHalf* const BP[], int ldb, const hipblasHalf* beta,
                                    hipblasHalf* const CP[], int ldc, int batchCount) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm_batched(handle, VKBLAS_DT_F16, VKBLAS_DT_F16, 1, transA, transB, m, n, k, alpha,
                                         AP, lda, BP, ldb, beta, (void*)CP, ldc, batchCount);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasHgemmBatched,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int, int, int, const hipblasHalf*,
               const hipblasHalf* const*, int, const hipblasHalf* const*, int, const hipblasHalf*,
               hipblasHalf* const*, int, int),
              (handle, transA, transB, m, n, k, alpha, AP, lda, BP, ldb, beta, CP, ldc, batchCount));
}

hipblasStatus_t hipblasHgemmBatched_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                       hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                       const hipblasHalf* alpha, const hipblasHalf* const AP[], int64_t lda,
                                       const hipblasHalf* const BP[], int64_t ldb, const hipblasHalf* beta,
                                       hipblasHalf* const CP[], int64_t ldc, int64_t batchCount) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    hipblasStatus_t s = run_gemm_batched(handle, VKBLAS_DT_F16, VKBLAS_DT_F16, 1, transA, transB, m, n, k, alpha,
                                         AP, lda, BP, ldb, beta, (void*)CP, ldc, batchCount);
    if (s != VKB_DECLINE) return s;
    REAL_CALL(hipblasStatus_t, hipblasHgemmBatched_64,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int64_t, int64_t, int64_t,
               const hipblasHalf*, const hipblasHalf* const*, int64_t, const hipblasHalf* const*, int64_t,
               const hipblasHalf*, hipblasHalf* const*, int64_t, int64_t),
              (handle, transA, transB, m, n, k, alpha, AP, lda, BP, ldb, beta, CP, ldc, batchCount));
}

hipblasStatus_t hipblasGemmBatchedEx(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                     int m, int n, int k, const void* alpha, const void* A[], hipDataType aType,
                                     int lda, const void* B[], hipDataType bType, int ldb, const void* beta,
                                     void* C[], hipDataType cType, int ldc, int batchCount,
                                     hipblasComputeType_t computeType, hipblasGemmAlgo_t algo) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    vkblas_dtype_t ab, ct;
    int sf16;
    if (ex_types((int)aType, (int)bType, (int)cType, (int)computeType, &ab, &ct, &sf16)) {
        hipblasStatus_t s = run_gemm_batched(handle, ab, ct, sf16, transA, transB, m, n, k, alpha, A, lda, B, ldb,
                                             beta, C, ldc, batchCount);
        if (s != VKB_DECLINE) return s;
    }
    REAL_CALL(hipblasStatus_t, hipblasGemmBatchedEx,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int, int, int, const void*, const void**,
               hipDataType, int, const void**, hipDataType, int, const void*, void**, hipDataType, int, int,
               hipblasComputeType_t, hipblasGemmAlgo_t),
              (handle, transA, transB, m, n, k, alpha, A, aType, lda, B, bType, ldb, beta, C, cType, ldc, batchCount,
               computeType, algo));
}

hipblasStatus_t hipblasGemmBatchedEx_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                        hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                        const void* alpha, const void* A[], hipDataType aType, int64_t lda,
                                        const void* B[], hipDataType bType, int64_t ldb, const void* beta,
                                        void* C[], hipDataType cType, int64_t ldc, int64_t batchCount,
                                        hipblasComputeType_t computeType, hipblasGemmAlgo_t algo) {
    if (!handle) return HIPBLAS_STATUS_INVALID_VALUE;
    vkblas_dtype_t ab, ct;
    int sf16;
    if (ex_types((int)aType, (int)bType, (int)cType, (int)computeType, &ab, &ct, &sf16)) {
        hipblasStatus_t s = run_gemm_batched(handle, ab, ct, sf16, transA, transB, m, n, k, alpha, A, lda, B, ldb,
                                             beta, C, ldc, batchCount);
        if (s != VKB_DECLINE) return s;
    }
    REAL_CALL(hipblasStatus_t, hipblasGemmBatchedEx_64,
              (hipblasHandle_t, hipblasOperation_t, hipblasOperation_t, int64_t, int64_t, int64_t, const void*,
               const void**, hipDataType, int64_t, const void**, hipDataType, int64_t, const void*, void**,
               hipDataType, int64_t, int64_t, hipblasComputeType_t, hipblasGemmAlgo_t),
              (handle, transA, transB, m, n, k, alpha, A, aType, lda, B, bType, ldb, beta, C, cType, ldc, batchCount,
               computeType, algo));
}

/* ------------------------------------------------ forward-only GEMMs */
/* fp64 / complex GEMMs: out of this build's scope; the reference also let the
 * real library handle them first or on failure (src/vkblas_hipblas.c:467-630). */

VKB_FWD(hipblasStatus_t, NS, hipblasDgemm, hipblasDgemm,
        (hipblasHandle_t h, hipblasOperation_t ta, hipblasOperation_t tb, int m, int n, int k, const double* al,
         const double* A, int lda, const double* B, int ldb, const double* be, double* C, int ldc),
        (h, ta, tb, m, n, k, al, A, lda, B, ldb, be, C, ldc))
VKB_FWD(hipblasStatus_t, NS, hipblasDgemmStridedBatched, hipblasDgemmStridedBatched,
        (hipblasHandle_t h, hipblasOperation_t ta, hipblasOperation_t tb, int m, int n, int k, const double* al,
         const double* A, int lda, long long sa, const double* B, int ldb, long long sb, const double* be,
         double* C, int ldc, long long sc, int bc),
        (h, ta, tb, m, n, k, al, A, lda, sa, B, ldb, sb, be, C, ldc, sc, bc))

#define VKB_CGEMM(name, real, T)                                                                            \
    VKB_FWD(hipblasStatus_t, NS, name, real,                                                                \
            (hipblasHandle_t h, hipblasOperation_t ta, hipblasOperation_t tb, int m, int n, int k,          \
             const T* al, const T* A, int lda, const T* B, int ldb, const T* be, T* C, int ldc),            \
            (h, ta, tb, m, n, k, al, A, lda, B, ldb, be, C, ldc))
#define VKB_CGEMM_SB(name, real, T)                                                                         \
    VKB_FWD(hipblasStatus_t, NS, name, real,                                                                \
            (hipblasHandle_t h, hipblasOperation_t ta, hipblasOperation_t tb, int m, int n, int k,          \
             const T* al, const T* A, int lda, long long sa, const T* B, int ldb, long long sb,              \
             const T* be, T* C, int ldc, long long sc, int bc),                                             \
            (h, ta, tb, m, n, k, al, A, lda, sa, B, ldb, sb, be, C, ldc, sc, bc))

VKB_CGEMM(hipblasCgemm, hipblasCgemm, hipComplex)
VKB_CGEMM(hipblasCgemm_v2, hipblasCgemm, hipComplex)
VKB_CGEMM(hipblasZgemm, hipblasZgemm, hipDoubleComplex)
VKB_CGEMM(hipblasZgemm_v2, hipblasZgemm, hipDoubleComplex)
VKB_CGEMM_SB(hipblasCgemmStridedBatched, hipblasCgemmStridedBatched, hipComplex)
VKB_CGEMM_SB(hipblasCgemmStridedBatched_v2, hipblasCgemmStridedBatched, hipComplex)
VKB_CGEMM_SB(hipblasZgemmStridedBatched, hipblasZgemmStridedBatched, hipDoubleComplex)
VKB_CGEMM_SB(hipblasZgemmStridedBatched_v2, hipblasZgemmStridedBatched, hipDoubleComplex)

/* ------------------------------------- dot / gemv / trsm / factorisations */
/* Forwarded unchanged (reference src/vkblas_hipblas.c:632-800).  The _v2
 * names of hipBLAS 2 map to hipBLAS 3's unsuffixed symbols. */

VKB_FWD(hipblasStatus_t, NS, hipblasSdot, hipblasSdot,
        (hipblasHandle_t h, int n, const float* x, int incx, const float* y, int incy, float* r),
        (h, n, x, incx, y, incy, r))
VKB_FWD(hipblasStatus_t, NS, hipblasDdot, hipblasDdot,
        (hipblasHandle_t h, int n, const double* x, int incx, const double* y, int incy, double* r),
        (h, n, x, incx, y, incy, r))
#define VKB_CDOT(name, real, T)                                                                             \
    VKB_FWD(hipblasStatus_t, NS, name, real,                                                                \
            (hipblasHandle_t h, int n, const T* x, int incx, const T* y, int incy, T* r),                   \
            (h, n, x, incx, y, incy, r))
VKB_CDOT(hipblasCdotc, hipblasCdotc, hipComplex)
VKB_CDOT(hipblasCdotc_v2, hipblasCdotc, hipComplex)
VKB_CDOT(hipblasCdotu, hipblasCdotu, hipComplex)
VKB_CDOT(hipblasCdotu_v2, hipblasCdotu, hipComplex)
VKB_CDOT(hipblasZdotc, hipblasZdotc, hipDoubleComplex)
VKB_CDOT(hipblasZdotc_v2, hipblasZdotc, hipDoubleComplex)
VKB_CDOT(hipblasZdotu, hipblasZdotu, hipDoubleComplex)
VKB_CDOT(hipblasZdotu_v2, hipblasZdotu, hipDoubleComplex)

#define VKB_DOTEX(name)                                                                                     \
    VKB_FWD(hipblasStatus_t, NS, name, hipblasDotEx,                                                        \
            (hipblasHandle_t h, int n, const void* x, hipDataType xt, int incx, const void* y,              \
             hipDataType yt, int incy, void* r, hipDataType rt, hipDataType et),                            \
            (h, n, x, xt, incx, y, yt, incy, r, rt, et))
VKB_DOTEX(hipblasDotEx)
VKB_DOTEX(hipblasDotEx_v2)

#define VKB_GEMV(name, real, T)                                                                             \
    VKB_FWD(hipblasStatus_t, NS, name, real,                                                                \
            (hipblasHandle_t h, hipblasOperation_t tr, int m, int n, const T* al, const T* A, int lda,      \
             const T* x, int incx, const T* be, T* y, int incy),                                            \
            (h, tr, m, n, al, A, lda, x, incx, be, y, incy))
VKB_GEMV(hipblasSgemv, hipblasSgemv, float)
VKB_GEMV(hipblasDgemv, hipblasDgemv, double)
VKB_GEMV(hipblasCgemv, hipblasCgemv, hipComplex)
VKB_GEMV(hipblasCgemv_v2, hipblasCgemv, hipComplex)
VKB_GEMV(hipblasZgemv, hipblasZgemv, hipDoubleComplex)
VKB_GEMV(hipblasZgemv_v2, hipblasZgemv, hipDoubleComplex)

#define VKB_TRSM(name, real, T)                                                                             \
    VKB_FWD(hipblasStatus_t, NS, name, real,                                                                \
            (hipblasHandle_t h, hipblasSideMode_t sd, hipblasFillMode_t ul, hipblasOperation_t ta,          \
             hipblasDiagType_t dg, int m, int n, const T* al, const T* A, int lda, T* B, int ldb),          \
            (h, sd, ul, ta, dg, m, n, al, A, lda, B, ldb))
VKB_TRSM(hipblasStrsm, hipblasStrsm, float)
VKB_TRSM(hipblasDtrsm, hipblasDtrsm, double)
VKB_TRSM(hipblasCtrsm, hipblasCtrsm, hipComplex)
VKB_TRSM(hipblasCtrsm_v2, hipblasCtrsm, hipComplex)
VKB_TRSM(hipblasZtrsm, hipblasZtrsm, hipDoubleComplex)
VKB_TRSM(hipblasZtrsm_v2, hipblasZtrsm, hipDoubleComplex)

#define VKB_TRSMB(name, real, T)                                                                            \
    VKB_FWD(hipblasStatus_t, NS, name, real,                                                                \
            (hipblasHandle_t h, hipblasSideMode_t sd, hipblasFillMode_t ul, hipblasOperation_t ta,          \
             hipblasDiagType_t dg, int m, int n, const T* al, const T* const A[], int lda, T* const B[],    \
             int ldb, int bc),                                                                              \
            (h, sd, ul, ta, dg, m, n, al, A, lda, B, ldb, bc))
VKB_TRSMB(hipblasStrsmBatched, hipblasStrsmBatched, float)
VKB_TRSMB(hipblasDtrsmBatched, hipblasDtrsmBatched, double)
VKB_TRSMB(hipblasCtrsmBatched, hipblasCtrsmBatched, hipComplex)
VKB_TRSMB(hipblasCtrsmBatched_v2, hipblasCtrsmBatched, hipComplex)
VKB_TRSMB(hipblasZtrsmBatched, hipblasZtrsmBatched, hipDoubleComplex)
VKB_TRSMB(hipblasZtrsmBatched_v2, hipblasZtrsmBatched, hipDoubleComplex)

#define VKB_GELS(name, real, T)                                                                             \
    VKB_FWD(hipblasStatus_t, NS, name, real,                                                                \
            (hipblasHandle_t h, hipblasOperation_t tr, const int m, const int n, const int nrhs,            \
             T* const A[], const int lda, T* const B[], const int ldb, int* info, int* dinfo,               \
             const int bc),                                                                                 \
            (h, tr, m, n, nrhs, A, lda, B, ldb, info, dinfo, bc))
VKB_GELS(hipblasSgelsBatched, hipblasSgelsBatched, float)
VKB_GELS(hipblasDgelsBatched, hipblasDgelsBatched, double)
VKB_GELS(hipblasCgelsBatched, hipblasCgelsBatched, hipComplex)
VKB_GELS(hipblasCgelsBatched_v2, hipblasCgelsBatched, hipComplex)
VKB_GELS(hipblasZgelsBatched, hipblasZgelsBatched, hipDoubleComplex)
VKB_GELS(hipblasZgelsBatched_v2, hipblasZgelsBatched, hipDoubleComplex)

#define VKB_GEQRF(name, real, T)                                                                            \
    VKB_FWD(hipblasStatus_t, NS, name, real,                                                                \
            (hipblasHandle_t h, const int m, const int n, T* const A[], const int lda, T* const ipiv[],     \
             int* info, const int bc),                                                                      \
            (h, m, n, A, lda, ipiv, info, bc))
VKB_GEQRF(hipblasSgeqrfBatched, hipblasSgeqrfBatched, float)
VKB_GEQRF(hipblasDgeqrfBatched, hipblasDgeqrfBatched, double)
VKB_GEQRF(hipblasCgeqrfBatched, hipblasCgeqrfBatched, hipComplex)
VKB_GEQRF(hipblasCgeqrfBatched_v2, hipblasCgeqrfBatched, hipComplex)
VKB_GEQRF(hipblasZgeqrfBatched, hipblasZgeqrfBatched, hipDoubleComplex)
VKB_GEQRF(hipblasZgeqrfBatched_v2, hipblasZgeqrfBatched, hipDoubleComplex)

#define VKB_GETRF(name, real, T)                                                                            \
    VKB_FWD(hipblasStatus_t, NS, name, real,                                                                \
            (hipblasHandle_t h, const int n, T* const A[], const int lda, int* ipiv, int* info,             \
             const int bc),                                                                                 \
            (h, n, A, lda, ipiv, info, bc))
VKB_GETRF(hipblasSgetrfBatched, hipblasSgetrfBatched, float)
VKB_GETRF(hipblasDgetrfBatched, hipblasDgetrfBatched, double)
VKB_GETRF(hipblasCgetrfBatched, hipblasCgetrfBatched, hipComplex)
VKB_GETRF(hipblasCgetrfBatched_v2, hipblasCgetrfBatched, hipComplex)
VKB_GETRF(hipblasZgetrfBatched, hipblasZgetrfBatched, hipDoubleComplex)
VKB_GETRF(hipblasZgetrfBatched_v2, hipblasZgetrfBatched, hipDoubleComplex)

#define VKB_GETRS(name, real, T)                                                                            \
    VKB_FWD(hipblasStatus_t, NS, name, real,                                                                \
            (hipblasHandle_t h, const hipblasOperation_t tr, const int n, const int nrhs, T* const A[],     \
             const int lda, const int* ipiv, T* const B[], const int ldb, int* info, const int bc),         \
            (h, tr, n, nrhs, A, lda, ipiv, B, ldb, info, bc))
VKB_GETRS(hipblasSgetrsBatched, hipblasSgetrsBatched, float)
VKB_GETRS(hipblasDgetrsBatched, hipblasDgetrsBatched, double)
VKB_GETRS(hipblasCgetrsBatched, hipblasCgetrsBatched, hipComplex)
VKB_GETRS(hipblasCgetrsBatched_v2, hipblasCgetrsBatched, hipComplex)
VKB_GETRS(hipblasZgetrsBatched, hipblasZgetrsBatched, hipDoubleComplex)
VKB_GETRS(hipblasZgetrsBatched_v2, hipblasZgetrsBatched, hipDoubleComplex)
