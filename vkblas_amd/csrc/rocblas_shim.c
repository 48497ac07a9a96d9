/*
 * rocblas_shim.c — rocBLAS GEMM entry points of libvkblas_hipblas.so (C11).
 *
 * PyTorch-ROCm computes fp16 / bf16 GEMMs through rocblas_gemm_ex and
 * rocblas_gemm_strided_batched_ex on its hipBLAS handle, so the drop-in
 * interposes them as the reference does (src/vkblas_hipblas.c:802-955).  The
 * call is translated to the row-major engine exactly as at the hipBLAS layer:
 * rocBLAS D(m x n) = alpha op(A) op(B) + beta C, column-major, is the
 * row-major D'(n x m) = op(B)' op(A)', so the engine runs with
 *     op_a = transB, op_b = transA, M = n, N = m, A = b, lda = ldb, B = a, ldb = lda.
 *
 * Differences from the reference, on purpose:
 *   - asynchronous on the handle's stream (rocblas_get_stream), no host sync
 *     (reference line 867);
 *   - rocblas_pointer_mode_device scalars are read by the kernels;
 *   - a D distinct from C is supported (the kernels read beta's matrix from
 *     C and write D; with beta == 0 C is never read); the reference
 *     forwarded c != d (line 838);
 *   - fp16 inputs with fp32 C / D are computed too;
 *   - m, n, k or batch_count <= 0 and invalid leading dimensions are forwarded
 *     so rocBLAS's own quick-return and error semantics apply (the reference
 *     returned invalid_value, line 836);
 *   - bf16 inputs with bf16 or fp32 C / D are computed (the reference
 *     forwarded rocBLAS bf16 calls);
 *   - the real library is found among the libraries the process already
 *     loaded (RTLD_NEXT, then librocblas.so.5 by soname), not by dlopen of a
 *     fixed path (reference lines 811-819).
 */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <hip/hip_runtime_api.h>

#include "vkblas_ext.h"
#include "vkblas_rocblas.h"

/* ------------------------------------------------------ real rocBLAS lookup */

static pthread_once_t g_once = PTHREAD_ONCE_INIT;
static void* g_real = NULL;
static void* g_self_base = NULL;
static int g_trace = 0;

static void self_anchor(void) {}

static int in_self(void* f) {
    Dl_info info;
    if (!f || !dladdr(f, &info)) return 0;
    return info.dli_fbase == g_self_base;
}

static void real_open(void) {
    Dl_info info;
    const char* e = getenv("VKBLAS_TRACE");
    g_trace = e && e[0] && e[0] != '0';
    if (dladdr((void*)&self_anchor, &info)) g_self_base = info.dli_fbase;
    static const char* names[] = {"librocblas.so.5", "librocblas.so", "/opt/rocm/lib/librocblas.so.5"};
    const int n = (int)(sizeof(names) / sizeof(names[0]));
    /* the instance the process already uses first; load one only if none is */
    for (int pass = 0; pass < 2 && !g_real; ++pass) {
        for (int i = 0; i < n && !g_real; ++i) {
            void* h = dlopen(names[i], RTLD_LAZY | (pass == 0 ? RTLD_NOLOAD : RTLD_LOCAL));
            if (!h) continue;
            void* probe = dlsym(h, "rocblas_get_stream");
            if (probe && !in_self(probe)) g_real = h;
            else dlclose(h);
        }
    }
    if (!g_real && g_trace) fprintf(stderr, "[vkblas] real librocblas not found: forwarding disabled\n");
}

/* A symbol of the real rocBLAS; never one of this library's. */
static void* real_sym(const char* name) {
    pthread_once(&g_once, real_open);
    void* f = dlsym(RTLD_NEXT, name);
    if (f && !in_self(f)) return f;
    if (g_real) {
        f = dlsym(g_real, name);
        if (f && !in_self(f)) return f;
    }
    return NULL;
}

static void* cached_sym(void** slot, const char* name) {
    void* f = __atomic_load_n(slot, __ATOMIC_ACQUIRE);
    if (!f) {
        f = real_sym(name);
        __atomic_store_n(slot, f, __ATOMIC_RELEASE);
    }
    return f;
}

/* ---------------------------------------------------------------- the GEMM */

typedef struct {
    rocblas_handle handle;
    rocblas_operation transA, transB;
    int64_t m, n, k;
    const void* alpha;
    const void* a;
    rocblas_datatype a_type;
    int64_t lda, sa;
    const void* b;
    rocblas_datatype b_type;
    int64_t ldb, sb;
    const void* beta;
    const void* c;
    rocblas_datatype c_type;
    int64_t ldc, sc;
    void* d;
    rocblas_datatype d_type;
    int64_t ldd, sd;
    int64_t batch;
    rocblas_datatype compute_type;
    uint32_t flags;
    int ptr_array;   /* a, b, c, d: device arrays of batch matrix pointers */
} gemm_call;

static int op_t(rocblas_operation op) {
    return op == rocblas_operation_transpose || op == rocblas_operation_conjugate_transpose;
}

static const char* dtype_name(vkblas_dtype_t t) {
    return t == VKBLAS_DT_F16 ? "f16" : t == VKBLAS_DT_BF16 ? "bf16" : "f32";
}

static int dtype_of(rocblas_datatype t, vkblas_dtype_t* out) {
    if (t == rocblas_datatype_f32_r) { *out = VKBLAS_DT_F32; return 1; }
    if (t == rocblas_datatype_f16_r) { *out = VKBLAS_DT_F16; return 1; }
    if (t == rocblas_datatype_bf16_r) { *out = VKBLAS_DT_BF16; return 1; }
    return 0;
}

/* 0 = computed; 1 = declined (the caller forwards); 2 = failed after part
 * of D was written (the caller reports it and does not forward). */
static int run(const gemm_call* g) {
    pthread_once(&g_once, real_open);
    if (!g->handle || !g->alpha || !g->beta || !g->a || !g->b || !g->d) return 1;
    if (g->m <= 0 || g->n <= 0 || g->k <= 0 || g->batch <= 0) return 1;
    if (g->m > UINT32_MAX || g->n > UINT32_MAX || g->k > UINT32_MAX || g->batch > UINT32_MAX) return 1;
    if (g->lda > UINT32_MAX || g->ldb > UINT32_MAX || g->ldc > UINT32_MAX || g->ldd > UINT32_MAX) return 1;
    if (g->lda < (op_t(g->transA) ? g->k : g->m) || g->ldb < (op_t(g->transB) ? g->n : g->k)) return 1;
    if (g->ldc < g->m || g->ldd < g->m) return 1;
    if (g->c == g->d && (g->ldc != g->ldd || g->sc != g->sd)) return 1;
    if (g->compute_type != rocblas_datatype_f32_r) return 1;
    /* solution-index queries and stochastic rounding stay with rocBLAS;
     * the fp16 alternate-implementation flags only affect rocBLAS's own
     * internal rounding of fp16 products, which fp32 MFMA accumulation
     * does not have */
    if (g->flags & ~(uint32_t)(rocblas_gemm_flags_use_cu_efficiency | rocblas_gemm_flags_fp16_alt_impl |
                               rocblas_gemm_flags_fp16_alt_impl_rnz))
        return 1;
    vkblas_dtype_t ab, cb, ct, dt;
    if (!dtype_of(g->a_type, &ab) || !dtype_of(g->b_type, &cb) || ab != cb) return 1;
    if (!dtype_of(g->c_type, &ct) || !dtype_of(g->d_type, &dt) || ct != dt) return 1;

    hipStream_t stream = NULL;
    rocblas_pointer_mode mode = rocblas_pointer_mode_host;
    static void* gs_fn;
    static void* gm_fn;
    void* gs = cached_sym(&gs_fn, "rocblas_get_stream");
    void* gm = cached_sym(&gm_fn, "rocblas_get_pointer_mode");
    if (!gs || !gm) return 1;
    if (((rocblas_status(*)(rocblas_handle, hipStream_t*))gs)(g->handle, &stream) != rocblas_status_success) return 1;
    if (((rocblas_status(*)(rocblas_handle, rocblas_pointer_mode*))gm)(g->handle, &mode) != rocblas_status_success)
        return 1;

    float alpha = 0.0f, beta = 0.0f;
    vkblas_scalar_mode_t sm = VKBLAS_SCALAR_HOST;
    const void* ad = NULL;
    const void* bd = NULL;
    int beta_maybe_nonzero = 1;
    if (mode == rocblas_pointer_mode_device) {
        sm = VKBLAS_SCALAR_DEV_F32;
        ad = g->alpha;
        bd = g->beta;
    } else {
        alpha = *(const float*)g->alpha;
        beta = *(const float*)g->beta;
        beta_maybe_nonzero = beta != 0.0f;
    }
    if (g_trace)
        fprintf(stderr, "[vkblas] rocblas gemm %s%s %s->%s m=%lld n=%lld k=%lld lda=%lld ldb=%lld ldc=%lld ldd=%lld "
                        "batch=%lld\n",
                op_t(g->transA) ? "T" : "N", op_t(g->transB) ? "T" : "N", dtype_name(ab), dtype_name(ct),
                (long long)g->m, (long long)g->n, (long long)g->k,
                (long long)g->lda, (long long)g->ldb, (long long)g->ldc, (long long)g->ldd, (long long)g->batch);

    /* D separate from C: the kernels read beta's matrix from C and write D
     * (with pointer arrays the matrices are not known on the host: declined) */
    if (g->ptr_array && g->c != g->d) return 1;
    vkblas_epilogue_t epi;
    memset(&epi, 0, sizeof(epi));
    if (!g->ptr_array && g->c != g->d && beta_maybe_nonzero) {
        if (!g->c) return 1;
        epi.c_in = g->c;
        epi.ldc_in = (uint32_t)g->ldc;
        epi.stride_c_in = g->batch > 1 ? g->sc : 0;
    }
    const vkblas_op_t op_a = op_t(g->transB) ? VKBLAS_OP_T : VKBLAS_OP_N;
    const vkblas_op_t op_b = op_t(g->transA) ? VKBLAS_OP_T : VKBLAS_OP_N;
    vkblas_status_t st;
    if (g->ptr_array)
        st = vkblas_gemm_batched_async(ab, ct, op_a, op_b, (uint32_t)g->n, (uint32_t)g->m, (uint32_t)g->k, alpha,
                                       (const void* const*)g->b, (uint32_t)g->ldb, (const void* const*)g->a,
                                       (uint32_t)g->lda, beta, (void* const*)g->d, (uint32_t)g->ldd,
                                       (uint32_t)g->batch, sm, ad, bd, stream);
    else
        st = vkblas_gemm_ex_async(ab, ct, op_a, op_b, (uint32_t)g->n, (uint32_t)g->m, (uint32_t)g->k, alpha, g->b,
                                  (uint32_t)g->ldb, g->a, (uint32_t)g->lda, beta, g->d, (uint32_t)g->ldd,
                                  (uint32_t)g->batch, g->batch > 1 ? g->sb : 0, g->batch > 1 ? g->sa : 0,
                                  g->batch > 1 ? g->sd : 0, sm, ad, bd, 0, epi.c_in ? &epi : NULL, stream);
    if (st == VKBLAS_ERR_PARTIAL) {
        if (g_trace) fprintf(stderr, "[vkblas] engine status %d: execution failed, not forwarded\n", (int)st);
        return 2;
    }
    if (st != VKBLAS_OK) {
        if (g_trace) fprintf(stderr, "[vkblas] engine status %d: forwarding\n", (int)st);
        return 1;
    }
    return 0;
}

/* ------------------------------------------------------------ entry points */

typedef rocblas_status (*gemm_ex_t)(rocblas_handle, rocblas_operation, rocblas_operation, rocblas_int, rocblas_int,
                                    rocblas_int, const void*, const void*, rocblas_datatype, rocblas_int,
                                    const void*, rocblas_datatype, rocblas_int, const void*, const void*,
                                    rocblas_datatype, rocblas_int, void*, rocblas_datatype, rocblas_int,
                                    rocblas_datatype, rocblas_gemm_algo, int32_t, uint32_t);
typedef rocblas_status (*gemm_ex64_t)(rocblas_handle, rocblas_operation, rocblas_operation, int64_t, int64_t,
                                      int64_t, const void*, const void*, rocblas_datatype, int64_t, const void*,
                                      rocblas_datatype, int64_t, const void*, const void*, rocblas_datatype,
                                      int64_t, void*, rocblas_datatype, int64_t, rocblas_datatype,
                                      rocblas_gemm_algo, int32_t, uint32_t);
typedef rocblas_status (*gemm_sb_t)(rocblas_handle, rocblas_operation, rocblas_operation, rocblas_int, rocblas_int,
                                    rocblas_int, const void*, const void*, rocblas_datatype, rocblas_int,
                                    rocblas_stride, const void*, rocblas_datatype, rocblas_int, rocblas_stride,
                                    const void*, const void*, rocblas_datatype, rocblas_int, rocblas_stride, void*,
                                    rocblas_datatype, rocblas_int, rocblas_stride, rocblas_int, rocblas_datatype,
                                    rocblas_gemm_algo, int32_t, uint32_t);
typedef rocblas_status (*gemm_sb64_t)(rocblas_handle, rocblas_operation, rocblas_operation, int64_t, int64_t,
                                      int64_t, const void*, const void*, rocblas_datatype, int64_t,
                                      rocblas_stride, const void*, rocblas_datatype, int64_t, rocblas_stride,
                                      const void*, const void*, rocblas_datatype, int64_t, rocblas_stride, void*,
                                      rocblas_datatype, int64_t, rocblas_stride, int64_t, rocblas_datatype,
                                      rocblas_gemm_algo, int32_t, uint32_t);

rocblas_status(rocblas_gemm_ex)(rocblas_handle handle, rocblas_operation transA, rocblas_operation transB,
                                rocblas_int m, rocblas_int n, rocblas_int k, const void* alpha, const void* a,
                                rocblas_datatype a_type, rocblas_int lda, const void* b, rocblas_datatype b_type,
                                rocblas_int ldb, const void* beta, const void* c, rocblas_datatype c_type,
                                rocblas_int ldc, void* d, rocblas_datatype d_type, rocblas_int ldd,
                                rocblas_datatype compute_type, rocblas_gemm_algo algo, int32_t solution_index,
                                uint32_t flags) {
    const gemm_call g = {handle, transA, transB, m, n, k, alpha, a, a_type, lda, 0, b, b_type, ldb, 0, beta,
                         c, c_type, ldc, 0, d, d_type, ldd, 0, 1, compute_type, flags, 0};
    const int r = run(&g);
    if (r == 0) return rocblas_status_success;
    if (r == 2) return rocblas_status_internal_error;
    static void* fn;
    gemm_ex_t f = (gemm_ex_t)cached_sym(&fn, "rocblas_gemm_ex");
    if (!f) return rocblas_status_not_implemented;
    return f(handle, transA, transB, m, n, k, alpha, a, a_type, lda, b, b_type, ldb, beta, c, c_type, ldc, d,
             d_type, ldd, compute_type, algo, solution_index, flags);
}

rocblas_status(rocblas_gemm_ex_64)(rocblas_handle handle, rocblas_operation transA, rocblas_operation transB,
                                   int64_t m, int64_t n, int64_t k, const void* alpha, const void* a,
                                   rocblas_datatype a_type, int64_t lda, const void* b, rocblas_datatype b_type,
                                   int64_t ldb, const void* beta, const void* c, rocblas_datatype c_type,
                                   int64_t ldc, void* d, rocblas_datatype d_type, int64_t ldd,
                                   rocblas_datatype compute_type, rocblas_gemm_algo algo, int32_t solution_index,
                                   uint32_t flags) {
    const gemm_call g = {handle, transA, transB, m, n, k, alpha, a, a_type, lda, 0, b, b_type, ldb, 0, beta,
                         c, c_type, ldc, 0, d, d_type, ldd, 0, 1, compute_type, flags, 0};
    const int r = run(&g);
    if (r == 0) return rocblas_status_success;
    if (r == 2) return rocblas_status_internal_error;
    static void* fn;
    gemm_ex64_t f = (gemm_ex64_t)cached_sym(&fn, "rocblas_gemm_ex_64");
    if (!f) return rocblas_status_not_implemented;
    return f(handle, transA, transB, m, n, k, alpha, a, a_type, lda, b, b_type, ldb, beta, c, c_type, ldc, d,
             d_type, ldd, compute_type, algo, solution_index, flags);
}

rocblas_status(rocblas_gemm_strided_batched_ex)(
    rocblas_handle handle, rocblas_operation transA, rocblas_operation transB, rocblas_int m, rocblas_int n,
    rocblas_int k, const void* alpha, const void* a, rocblas_datatype a_type, rocblas_int lda,
    rocblas_stride stride_a, const void* b, rocblas_datatype b_type, rocblas_int ldb, rocblas_stride stride_b,
    const void* beta, const void* c, rocblas_datatype c_type, rocblas_int ldc, rocblas_stride stride_c, void* d,
    rocblas_datatype d_type, rocblas_int ldd, rocblas_stride stride_d, rocblas_int batch_count,
    rocblas_datatype compute_type, rocblas_gemm_algo algo, int32_t solution_index, uint32_t flags) {
    const gemm_call g = {handle, transA, transB, m, n, k, alpha, a, a_type, lda, stride_a, b, b_type, ldb,
                         stride_b, beta, c, c_type, ldc, stride_c, d, d_type, ldd, stride_d, batch_count,
                         compute_type, flags, 0};
    const int r = run(&g);
    if (r == 0) return rocblas_status_success;
    if (r == 2) return rocblas_status_internal_error;
    static void* fn;
    gemm_sb_t f = (gemm_sb_t)cached_sym(&fn, "rocblas_gemm_strided_batched_ex");
    if (!f) return rocblas_status_not_implemented;
    return f(handle, transA, transB, m, n, k, alpha, a, a_type, lda, stride_a, b, b_type, ldb, stride_b, beta, c,
             c_type, ldc, stride_c, d, d_type, ldd, stride_d, batch_count, compute_type, algo, solution_index,
             flags);
}

rocblas_status(rocblas_gemm_strided_batched_ex_64)(
    rocblas_handle handle, rocblas_operation transA, rocblas_operation transB, int64_t m, int64_t n, int64_t k,
    const void* alpha, const void* a, rocblas_datatype a_type, int64_t lda, rocblas_stride stride_a,
    const void* b, rocblas_datatype b_type, int64_t ldb, rocblas_stride stride_b, const void* beta,
    const void* c, rocblas_datatype c_type, int64_t ldc, rocblas_stride stride_c, void* d,
    rocblas_datatype d_type, int64_t ldd, rocblas_stride stride_d, int64_t batch_count,
    rocblas_datatype compute_type, rocblas_gemm_algo algo, int32_t solution_index, uint32_t flags) {
    const gemm_call g = {handle, transA, transB, m, n, k, alpha, a, a_type, lda, stride_a, b, b_type, ldb,
                         stride_b, beta, c, c_type, ldc, stride_c, d, d_type, ldd, stride_d, batch_count,
                         compute_type, flags, 0};
    const int r = run(&g);
    if (r == 0) return rocblas_status_success;
    if (r == 2) return rocblas_status_internal_error;
    static void* fn;
    gemm_sb64_t f = (gemm_sb64_t)cached_sym(&fn, "rocblas_gemm_strided_batched_ex_64");
    if (!f) return rocblas_status_not_implemented;
    return f(handle, transA, transB, m, n, k, alpha, a, a_type, lda, stride_a, b, b_type, ldb, stride_b, beta, c,
             c_type, ldc, stride_c, d, d_type, ldd, stride_d, batch_count, compute_type, algo, solution_index,
             flags);
}

/* Pointer-array batched: no counterpart in the reference (it forwarded
 * rocblas_gemm_batched_ex).  a, b, c, d are device arrays of batch_count
 * matrix pointers; a separate D is declined. */
typedef rocblas_status (*gemm_b_t)(rocblas_handle, rocblas_operation, rocblas_operation, rocblas_int, rocblas_int,
                                   rocblas_int, const void*, const void*, rocblas_datatype, rocblas_int, const void*,
                                   rocblas_datatype, rocblas_int, const void*, const void*, rocblas_datatype,
                                   rocblas_int, void*, rocblas_datatype, rocblas_int, rocblas_int, rocblas_datatype,
                                   rocblas_gemm_algo, int32_t, uint32_t);
typedef rocblas_status (*gemm_b64_t)(rocblas_handle, rocblas_operation, rocblas_operation, int64_t, int64_t,
                                     int64_t, const void*, const void*, rocblas_datatype, int64_t, const void*,
                                     rocblas_datatype, int64_t, const void*, const void*, rocblas_datatype, int64_t,
                                     void*, rocblas_datatype, int64_t, int64_t, rocblas_datatype, rocblas_gemm_algo,
                                     int32_t, uint32_t);

rocblas_status(rocblas_gemm_batched_ex)(rocblas_handle handle, rocblas_operation transA, rocblas_operation transB,
                                        rocblas_int m, rocblas_int n, rocblas_int k, const void* alpha,
                                        const void* a, rocblas_datatype a_type, rocblas_int lda, const void* b,
                                        rocblas_datatype b_type, rocblas_int ldb, const void* beta, const void* c,
                                        rocblas_datatype c_type, rocblas_int ldc, void* d, rocblas_datatype d_type,
                                        rocblas_int ldd, rocblas_int batch_count, rocblas_datatype compute_type,
                                        rocblas_gemm_algo algo, int32_t solution_index, uint32_t flags) {
    const gemm_call g = {handle, transA, transB, m, n, k, alpha, a, a_type, lda, 0, b, b_type, ldb, 0, beta,
                         c, c_type, ldc, 0, d, d_type, ldd, 0, batch_count, compute_type, flags, 1};
    const int r = run(&g);
    if (r == 0) return rocblas_status_success;
    if (r == 2) return rocblas_status_internal_error;
    static void* fn;
    gemm_b_t f = (gemm_b_t)cached_sym(&fn, "rocblas_gemm_batched_ex");
    if (!f) return rocblas_status_not_implemented;
    return f(handle, transA, transB, m, n, k, alpha, a, a_type, lda, b, b_type, ldb, beta, c, c_type, ldc, d,
             d_type, ldd, batch_count, compute_type, algo, solution_index, flags);
}

rocblas_status(rocblas_gemm_batched_ex_64)(rocblas_handle handle, rocblas_operation transA,
                                           rocblas_operation transB, int64_t m, int64_t n, int64_t k,
                                           const void* alpha, const void* a, rocblas_datatype a_type, int64_t lda,
                                           const void* b, rocblas_datatype b_type, int64_t ldb, const void* beta,
                                           const void* c, rocblas_datatype c_type, int64_t ldc, void* d,
                                           rocblas_datatype d_type, int64_t ldd, int64_t batch_count,
                                           rocblas_datatype compute_type, rocblas_gemm_algo algo,
                                           int32_t solution_index, uint32_t flags) {
    const gemm_call g = {handle, transA, transB, m, n, k, alpha, a, a_type, lda, 0, b, b_type, ldb, 0, beta,
                         c, c_type, ldc, 0, d, d_type, ldd, 0, batch_count, compute_type, flags, 1};
    const int r = run(&g);
    if (r == 0) return rocblas_status_success;
    if (r == 2) return rocblas_status_internal_error;
    static void* fn;
    gemm_b64_t f = (gemm_b64_t)cached_sym(&fn, "rocblas_gemm_batched_ex_64");
    if (!f) return rocblas_status_not_implemented;
    return f(handle, transA, transB, m, n, k, alpha, a, a_type, lda, b, b_type, ldb, beta, c, c_type, ldc, d,
             d_type, ldd, batch_count, compute_type, algo, solution_index, flags);
}
