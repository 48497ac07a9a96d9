/*
 * oracle/ref_gemm.c — CPU restatement of the reference's GEMM oracles.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this code, and only as the checker
 * or the timed CPU comparator; the library never calls it and has no CPU
 * fallback.
 *
 * Functions and the reference code each one follows:
 *   oracle_ref_gemm_cm     test/test_gemm.c:32-58  (ref_gemm): hipBLAS
 *                          column-major semantics, double accumulation,
 *                          C = alpha * (float)s + beta * C, optional uniform
 *                          row sampling (rows r*m/sample, last row m-1).
 *   oracle_fill_test_gemm  test/test_gemm.c:70-73: srand(seed), then A, B, C
 *                          filled with (rand() % 200 - 100) / 10.0f.
 *   oracle_ref_gemm_f16_rm test/test_h.c:63-79 (cpu_ref, fp16 branch):
 *                          row-major engine contract on fp16 bit patterns,
 *                          double accumulation, old C read only if beta != 0,
 *                          result rounded to fp16.  Rounding here is IEEE
 *                          round-to-nearest-even (the reference's own f2h,
 *                          test/test_h.c:23-41, rounds ties up; the GPU
 *                          kernels round to nearest even, so the oracle does).
 *   oracle_ref_gemm_f32_rm fp32 on the row-major engine contract
 *                          (src/vkblas.h:21-26): same arithmetic as
 *                          oracle_ref_gemm_cm, except that beta == 0 never
 *                          reads C.  oracle_ref_gemm_cm keeps the reference's
 *                          beta * C term even for beta == 0, as ref_gemm does.
 *   oracle_ref_gemm_f16f32_rm  as oracle_ref_gemm_f16_rm with an fp32 result (GemmEx 16F->32F;
 *                          no reference counterpart, same arithmetic).
 *   oracle_fill_test_h     test/test_h.c:102, 111-113: after srand(seed),
 *                          values (float)rand()/RAND_MAX*2-1 converted to fp16
 *                          with ties rounded away from zero, which is what the
 *                          reference's f2h computes for these finite inputs.
 *   oracle_f2h_rne / oracle_h2f  IEEE binary16 conversions.
 *   oracle_bf2f / oracle_f2bf_rne  bfloat16 conversions as the reference's
 *                          shaders state them: bf16 -> fp32 is the bit
 *                          pattern shifted left 16
 *                          (src/shaders/gemm_half_128x128_bankfree_tmpl.comp:26-40),
 *                          fp32 -> bf16 rounds to nearest even
 *                          (same file :41-47, src/shaders/cvt_tmpl.comp:141).
 *                          NaN maps to a quiet NaN of the same sign; the
 *                          reference's integer rounding can carry a NaN with
 *                          a large payload into the sign bit, which nothing
 *                          in its tests exercises.
 *   oracle_ref_gemm_bf16_rm / oracle_ref_gemm_bf16f32_rm  the bf16 GEMM of
 *                          src/vkblas.c:3345-3512 (gemm_bf16_core: bf16
 *                          inputs, fp32 arithmetic, one bf16 rounding) on the
 *                          row-major engine contract, with the arithmetic of
 *                          oracle_ref_gemm_f16_rm (double accumulation of the
 *                          exact products, then alpha * (float)s + beta * C).
 *
 *   oracle_ref_gemm_epi_rm  any of the above input / output types (fp32, fp16,
 *                          bf16) with the epilogue hipBLASLt defines for its
 *                          HIPBLASLT_EPILOGUE_BIAS and its separate C and D
 *                          (no reference counterpart; PyTorch's addmm with a
 *                          1-D bias, reference test/test_torch.py:65-73,
 *                          reaches it): D = alpha * (float)s + beta * C_in +
 *                          bias[n], in fp32, rounded once to D's type; C_in
 *                          read only if beta != 0; bias (fp32 values, or
 *                          NULL) indexed by the column n of the row-major
 *                          result.  Without bias and with C_in == D it is the
 *                          functions above, bit for bit.
 * The *_omp variants split the same arithmetic over output columns with
 * OpenMP (each output is still computed by one thread in the same order).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------ fp16 bits */

float oracle_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else { /* subnormal: value = man * 2^-24 */
            int e = 0;
            while (!(man & 0x400u)) { man <<= 1; ++e; }
            u = sign | ((uint32_t)(113 - e) << 23) | ((man & 0x3ffu) << 13);
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

/* f32 -> f16 with rounding mode: 0 = nearest-even, 1 = nearest, ties away from zero */
static uint16_t f2h_mode(float f, int ties_away) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t exp = (u >> 23) & 0xffu, man = u & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int e = (int)exp - 127; /* unbiased */
    if (e > 15) return (uint16_t)(sign | 0x7c00u);
    uint32_t full = man | (exp ? 0x800000u : 0u); /* 24-bit significand */
    /* value = full * 2^(e-23) (exp != 0).  Target quantum: 2^-24 for
     * subnormal halves (e < -14), else 2^(e-10). */
    int shift; /* bits of full dropped */
    if (exp == 0) return sign; /* f32 subnormals are far below half's range */
    if (e < -14) shift = 13 + (-14 - e); else shift = 13;
    if (shift > 24) return sign;
    uint32_t q = full >> shift;
    uint32_t rem = full & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (ties_away || (q & 1u)))) q++;
    uint32_t bits;
    if (e < -14) {
        bits = q; /* subnormal (may round up into the smallest normal: q = 0x400) */
    } else {
        /* q holds 1.man in 11 bits; a carry to 0x800 bumps the exponent */
        uint32_t he = (uint32_t)(e + 15);
        if (q & 0x800u) { q >>= 1; he++; }
        if (he >= 31) return (uint16_t)(sign | 0x7c00u);
        bits = (he << 10) | (q & 0x3ffu);
    }
    return (uint16_t)(sign | bits);
}

uint16_t oracle_f2h_rne(float f) { return f2h_mode(f, 0); }
uint16_t oracle_f2h_ties_away(float f) { return f2h_mode(f, 1); }

void oracle_f2h_rne_array(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f2h_rne(x[i]);
}
void oracle_h2f_array(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_h2f(x[i]);
}

/* ------------------------------------------------------------ bf16 bits */

float oracle_bf2f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t oracle_f2bf_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u); /* quiet NaN */
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

void oracle_f2bf_rne_array(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_f2bf_rne(x[i]);
}
void oracle_bf2f_array(const uint16_t* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = oracle_bf2f(x[i]);
}

/* ------------------------------------------------------------- generators */

void oracle_fill_test_gemm(unsigned seed, float* A, int64_t na, float* B, int64_t nb, float* C, int64_t nc) {
    srand(seed);
    for (int64_t i = 0; i < na; ++i) A[i] = (float)(rand() % 200 - 100) / 10.0f;
    for (int64_t i = 0; i < nb; ++i) B[i] = (float)(rand() % 200 - 100) / 10.0f;
    for (int64_t i = 0; i < nc; ++i) C[i] = (float)(rand() % 200 - 100) / 10.0f;
}

void oracle_fill_test_h(unsigned seed, uint16_t* A, int64_t na, uint16_t* B, int64_t nb, uint16_t* C,
                        int64_t nc) {
    srand(seed);
    for (int64_t i = 0; i < na; ++i) A[i] = oracle_f2h_ties_away((float)rand() / RAND_MAX * 2.0f - 1.0f);
    for (int64_t i = 0; i < nb; ++i) B[i] = oracle_f2h_ties_away((float)rand() / RAND_MAX * 2.0f - 1.0f);
    for (int64_t i = 0; i < nc; ++i) C[i] = oracle_f2h_ties_away((float)rand() / RAND_MAX * 2.0f - 1.0f);
}

/* ---------------------------------------------------- fp32 column-major */

/* rows[] gets the sampled row indices; returns their count */
int oracle_sample_rows(int m, int sample, int* rows) {
    if (sample <= 0 || sample >= m) {
        for (int i = 0; i < m; ++i) rows[i] = i;
        return m;
    }
    for (int r = 0; r < sample; ++r) rows[r] = (int)((int64_t)r * m / sample);
    rows[sample - 1] = m - 1;
    return sample;
}

static void ref_cm_col(int ta, int tb, int i, int j, int k, float alpha, const float* A, int64_t lda,
                       const float* B, int64_t ldb, float beta, float* C, int64_t ldc) {
    double s = 0.0;
    for (int t = 0; t < k; ++t) {
        float av = ta ? A[t + (int64_t)i * lda] : A[i + (int64_t)t * lda];
        float bv = tb ? B[j + (int64_t)t * ldb] : B[t + (int64_t)j * ldb];
        s += (double)av * bv;
    }
    C[i + (int64_t)j * ldc] = alpha * (float)s + beta * C[i + (int64_t)j * ldc];
}

/* ta / tb: 0 = N, 1 = T (hipBLAS transA / transB) */
void oracle_ref_gemm_cm_omp(int ta, int tb, int m, int n, int k, float alpha, const float* A, int64_t lda,
                            const float* B, int64_t ldb, float beta, float* C, int64_t ldc, int sample,
                            int threads) {
    int* rows = (int*)malloc(sizeof(int) * (size_t)(m > 0 ? m : 1));
    int nr = oracle_sample_rows(m, sample, rows);
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
    for (int j = 0; j < n; ++j)
        for (int ri = 0; ri < nr; ++ri) ref_cm_col(ta, tb, rows[ri], j, k, alpha, A, lda, B, ldb, beta, C, ldc);
    free(rows);
    (void)threads;
}

void oracle_ref_gemm_cm(int ta, int tb, int m, int n, int k, float alpha, const float* A, int64_t lda,
                        const float* B, int64_t ldb, float beta, float* C, int64_t ldc, int sample) {
    int* rows = (int*)malloc(sizeof(int) * (size_t)(m > 0 ? m : 1));
    int nr = oracle_sample_rows(m, sample, rows);
    for (int ri = 0; ri < nr; ++ri)
        for (int j = 0; j < n; ++j) ref_cm_col(ta, tb, rows[ri], j, k, alpha, A, lda, B, ldb, beta, C, ldc);
    free(rows);
}

/* ------------------------------------------------------ fp16 row-major */

/* 16-bit -> fp32 tables (filled before any parallel region) */
static float g_h2f_lut[65536];
static float g_bf2f_lut[65536];
static int g_h2f_ready = 0;
static void h2f_lut_init(void) {
    if (g_h2f_ready) return;
    for (uint32_t i = 0; i < 65536u; ++i) {
        g_h2f_lut[i] = oracle_h2f((uint16_t)i);
        g_bf2f_lut[i] = oracle_bf2f((uint16_t)i);
    }
    g_h2f_ready = 1;
}

static double dot_half(const float* lut, int op_a, int op_b, int m, int n, int K, const uint16_t* A,
                       int64_t lda, const uint16_t* B, int64_t ldb) {
    double s = 0.0;
    for (int k = 0; k < K; ++k) {
        float av = op_a ? lut[A[(int64_t)k * lda + m]] : lut[A[(int64_t)m * lda + k]];
        float bv = op_b ? lut[B[(int64_t)n * ldb + k]] : lut[B[(int64_t)k * ldb + n]];
        s += (double)av * bv;
    }
    return s;
}

/* Shared body of the 16-bit-input GEMMs.  bf != 0 selects bf16 inputs (and a
 * bf16 result when C16 is given); exactly one of C16 / C32 is non-NULL. */
static void ref_gemm_half_rm(int bf, int op_a, int op_b, int M, int N, int K, const uint16_t* A, int64_t lda,
                             const uint16_t* B, int64_t ldb, float alpha, float beta, uint16_t* C16, float* C32,
                             int64_t ldc, const int* rows, int nrows, int threads) {
    int nr = rows ? nrows : M;
    h2f_lut_init();
    const float* lut = bf ? g_bf2f_lut : g_h2f_lut;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for collapse(2) schedule(static) num_threads(threads)
#endif
    for (int ri = 0; ri < nr; ++ri) {
        for (int n = 0; n < N; ++n) {
            const int m = rows ? rows[ri] : ri;
            const int64_t at = (int64_t)m * ldc + n;
            double s = dot_half(lut, op_a, op_b, m, n, K, A, lda, B, ldb);
            if (C16) {
                float old = beta != 0.0f ? lut[C16[at]] : 0.0f;
                float v = alpha * (float)s + beta * old;
                C16[at] = bf ? oracle_f2bf_rne(v) : oracle_f2h_rne(v);
            } else {
                float old = beta != 0.0f ? C32[at] : 0.0f;
                C32[at] = alpha * (float)s + beta * old;
            }
        }
    }
    (void)threads;
}

/* op_a / op_b: engine ops (0 = N, 1 = T); rows: optional list of the rows m
 * to compute (NULL = all M) */
void oracle_ref_gemm_f16_rm(int op_a, int op_b, int M, int N, int K, const uint16_t* A, int64_t lda,
                            const uint16_t* B, int64_t ldb, float alpha, float beta, uint16_t* C, int64_t ldc,
                            const int* rows, int nrows, int threads) {
    ref_gemm_half_rm(0, op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, NULL, ldc, rows, nrows, threads);
}

void oracle_ref_gemm_f16f32_rm(int op_a, int op_b, int M, int N, int K, const uint16_t* A, int64_t lda,
                               const uint16_t* B, int64_t ldb, float alpha, float beta, float* C, int64_t ldc,
                               const int* rows, int nrows, int threads) {
    ref_gemm_half_rm(0, op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, NULL, C, ldc, rows, nrows, threads);
}

void oracle_ref_gemm_bf16_rm(int op_a, int op_b, int M, int N, int K, const uint16_t* A, int64_t lda,
                             const uint16_t* B, int64_t ldb, float alpha, float beta, uint16_t* C, int64_t ldc,
                             const int* rows, int nrows, int threads) {
    ref_gemm_half_rm(1, op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, NULL, ldc, rows, nrows, threads);
}

void oracle_ref_gemm_bf16f32_rm(int op_a, int op_b, int M, int N, int K, const uint16_t* A, int64_t lda,
                                const uint16_t* B, int64_t ldb, float alpha, float beta, float* C, int64_t ldc,
                                const int* rows, int nrows, int threads) {
    ref_gemm_half_rm(1, op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, NULL, C, ldc, rows, nrows, threads);
}

/* fp32 row-major engine contract (src/vkblas.h:21-26), same arithmetic as
 * oracle_ref_gemm_cm; used to check engine-API calls directly. */
void oracle_ref_gemm_f32_rm(int op_a, int op_b, int M, int N, int K, const float* A, int64_t lda, const float* B,
                            int64_t ldb, float alpha, float beta, float* C, int64_t ldc, const int* rows,
                            int nrows, int threads) {
    int nr = rows ? nrows : M;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for collapse(2) schedule(static) num_threads(threads)
#endif
    for (int ri = 0; ri < nr; ++ri) {
        for (int n = 0; n < N; ++n) {
            const int m = rows ? rows[ri] : ri;
            double s = 0.0;
            for (int k = 0; k < K; ++k) {
                float av = op_a ? A[(int64_t)k * lda + m] : A[(int64_t)m * lda + k];
                float bv = op_b ? B[(int64_t)n * ldb + k] : B[(int64_t)k * ldb + n];
                s += (double)av * bv;
            }
            float old = beta != 0.0f ? C[(int64_t)m * ldc + n] : 0.0f;
            C[(int64_t)m * ldc + n] = alpha * (float)s + beta * old;
        }
    }
    (void)threads;
}

/* Element types of oracle_ref_gemm_epi_rm: 0 fp32, 1 fp16, 2 bf16. */
static float load_t(int t, const void* p, int64_t i) {
    if (t == 0) return ((const float*)p)[i];
    h2f_lut_init();
    const uint16_t h = ((const uint16_t*)p)[i];
    return t == 1 ? g_h2f_lut[h] : g_bf2f_lut[h];
}

static void store_t(int t, void* p, int64_t i, float v) {
    if (t == 0) ((float*)p)[i] = v;
    else ((uint16_t*)p)[i] = t == 1 ? oracle_f2h_rne(v) : oracle_f2bf_rne(v);
}

void oracle_ref_gemm_epi_rm(int ab, int ct, int op_a, int op_b, int M, int N, int K, const void* A, int64_t lda,
                            const void* B, int64_t ldb, float alpha, float beta, const void* Cin, int64_t ldcin,
                            void* D, int64_t ldd, const float* bias, const int* rows, int nrows, int threads) {
    int nr = rows ? nrows : M;
    h2f_lut_init();
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for collapse(2) schedule(static) num_threads(threads)
#endif
    for (int ri = 0; ri < nr; ++ri) {
        for (int n = 0; n < N; ++n) {
            const int m = rows ? rows[ri] : ri;
            double s = 0.0;
            for (int k = 0; k < K; ++k) {
                float av = load_t(ab, A, op_a ? (int64_t)k * lda + m : (int64_t)m * lda + k);
                float bv = load_t(ab, B, op_b ? (int64_t)n * ldb + k : (int64_t)k * ldb + n);
                s += (double)av * bv;
            }
            float old = beta != 0.0f ? load_t(ct, Cin, (int64_t)m * ldcin + n) : 0.0f;
            float v = alpha * (float)s + beta * old;
            if (bias) v += bias[n];
            store_t(ct, D, (int64_t)m * ldd + n, v);
        }
    }
    (void)threads;
}

/* --------------------------------------------- tiled, bit for bit the same */

/* The arithmetic of oracle_ref_gemm_epi_rm (without bias, C_in == D) in an
 * order that caches: operands are converted to double once (A as [k][m], B
 * as [k][n]), and each thread keeps the double sums of a TM x TN block of C
 * while k runs.  Every output is still the sum s = s + a_k b_k for k = 0 ..
 * K-1 in that order, starting from 0 (the product of two floats is exact in
 * double either way; the build contracts nothing into fused multiply-adds):
 * the result equals the plain loops bit for bit (a test pins that).  For
 * full-output checks of large shapes, which the plain loops take minutes
 * over. */
void oracle_ref_gemm_tiled_rm(int ab, int ct, int op_a, int op_b, int M, int N, int K, const void* A, int64_t lda,
                              const void* B, int64_t ldb, float alpha, float beta, void* C, int64_t ldc,
                              int threads) {
    enum { TM = 64, TN = 256 };
    h2f_lut_init();
    double* Ad = (double*)malloc(sizeof(double) * (size_t)K * (size_t)M);
    double* Bd = (double*)malloc(sizeof(double) * (size_t)K * (size_t)N);
    if (!Ad || !Bd) {
        free(Ad);
        free(Bd);
        abort();
    }
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
#endif
    for (int k = 0; k < K; ++k) {
        for (int m = 0; m < M; ++m)
            Ad[(int64_t)k * M + m] = (double)load_t(ab, A, op_a ? (int64_t)k * lda + m : (int64_t)m * lda + k);
        for (int n = 0; n < N; ++n)
            Bd[(int64_t)k * N + n] = (double)load_t(ab, B, op_b ? (int64_t)n * ldb + k : (int64_t)k * ldb + n);
    }
    const int tm = (M + TM - 1) / TM, tn = (N + TN - 1) / TN;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
    for (int t = 0; t < tm * tn; ++t) {
        const int m0 = (t / tn) * TM, n0 = (t % tn) * TN;
        const int mc = M - m0 < TM ? M - m0 : TM, nc = N - n0 < TN ? N - n0 : TN;
        double* s = (double*)calloc((size_t)TM * TN, sizeof(double));
        if (!s) abort();
        for (int k = 0; k < K; ++k) {
            const double* a = Ad + (int64_t)k * M + m0;
            const double* b = Bd + (int64_t)k * N + n0;
            for (int i = 0; i < mc; ++i) {
                const double ai = a[i];
                double* si = s + (int64_t)i * TN;
#pragma omp simd
                for (int j = 0; j < nc; ++j) si[j] += ai * b[j];
            }
        }
        for (int i = 0; i < mc; ++i)
            for (int j = 0; j < nc; ++j) {
                const int64_t at = (int64_t)(m0 + i) * ldc + n0 + j;
                const float old = beta != 0.0f ? load_t(ct, C, at) : 0.0f;
                store_t(ct, C, at, alpha * (float)s[(int64_t)i * TN + j] + beta * old);
            }
        free(s);
    }
    free(Ad);
    free(Bd);
    (void)threads;
}
