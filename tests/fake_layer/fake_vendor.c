/*
 * fake_vendor.c — stand-ins for the vendor libraries (hipBLAS, rocBLAS) a
 * process would load, for the CPU tests of the drop-in library's forwarding.
 * Built once per soname (libhipblas.so.3, librocblas.so.5); each GEMM entry
 * point records which function was called and its arguments, so a test can
 * check that a call the engine declined reached the vendor unchanged.  No
 * GPU is used: the "handle" is an address the fake hands out.
 */
#include <stdint.h>
#include <string.h>

typedef struct {
    char fn[48];
    int calls;
    int ta, tb;
    int64_t m, n, k, lda, ldb, ldc, batch;
    const void *A, *B, *C;
    float alpha, beta;
} fake_call_t;

static fake_call_t g_last;
static int g_handle_storage;
static void* g_stream = (void*)0x5150;

const fake_call_t* fake_vendor_last(void) { return &g_last; }
void fake_vendor_reset(void) { memset(&g_last, 0, sizeof(g_last)); }

static void rec(const char* fn, int ta, int tb, int64_t m, int64_t n, int64_t k, const void* alpha, const void* A,
                int64_t lda, const void* B, int64_t ldb, const void* beta, const void* C, int64_t ldc,
                int64_t batch) {
    const int calls = g_last.calls + 1;
    memset(&g_last, 0, sizeof(g_last));
    strncpy(g_last.fn, fn, sizeof(g_last.fn) - 1);
    g_last.calls = calls;
    g_last.ta = ta; g_last.tb = tb;
    g_last.m = m; g_last.n = n; g_last.k = k;
    g_last.lda = lda; g_last.ldb = ldb; g_last.ldc = ldc; g_last.batch = batch;
    g_last.A = A; g_last.B = B; g_last.C = C;
    if (alpha) memcpy(&g_last.alpha, alpha, 4);
    if (beta) memcpy(&g_last.beta, beta, 4);
}

#ifdef FAKE_HIPBLAS
/* hipBLAS: statuses and enums by value (hipblasStatus_t 0 = success,
 * hipblasPointerMode_t 0 = host, hipblasOperation_t 111 / 112 = N / T) */
int hipblasCreate(void** handle) { *handle = &g_handle_storage; return 0; }
int hipblasDestroy(void* handle) { return 0; }
int hipblasSetStream(void* handle, void* s) { g_stream = s; return 0; }
int hipblasGetStream(void* handle, void** s) { *s = g_stream; return 0; }
int hipblasGetPointerMode(void* handle, int* mode) { *mode = 0; return 0; }
int hipblasSetPointerMode(void* handle, int mode) { return 0; }
int hipblasSgemm(void* h, int ta, int tb, int m, int n, int k, const float* alpha, const float* A, int lda,
                 const float* B, int ldb, const float* beta, float* C, int ldc) {
    rec("hipblasSgemm", ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, 1);
    return 0;
}
int hipblasSgemmStridedBatched(void* h, int ta, int tb, int m, int n, int k, const float* alpha, const float* A,
                               int lda, long long sA, const float* B, int ldb, long long sB, const float* beta,
                               float* C, int ldc, long long sC, int batch) {
    rec("hipblasSgemmStridedBatched", ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, batch);
    return 0;
}
int hipblasGemmEx(void* h, int ta, int tb, int m, int n, int k, const void* alpha, const void* A, int at, int lda,
                  const void* B, int bt, int ldb, const void* beta, void* C, int ct, int ldc, int comp, int algo) {
    rec("hipblasGemmEx", ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, 1);
    return 0;
}
int hipblasDgemm(void* h, int ta, int tb, int m, int n, int k, const double* alpha, const double* A, int lda,
                 const double* B, int ldb, const double* beta, double* C, int ldc) {
    rec("hipblasDgemm", ta, tb, m, n, k, NULL, A, lda, B, ldb, NULL, C, ldc, 1);
    return 0;
}
#endif

#ifdef FAKE_ROCBLAS
/* rocBLAS: rocblas_status 0 = success, rocblas_pointer_mode 0 = host,
 * rocblas_operation 111 / 112 = N / T */
int rocblas_create_handle(void** handle) { *handle = &g_handle_storage; return 0; }
int rocblas_destroy_handle(void* handle) { return 0; }
int rocblas_get_stream(void* handle, void** s) { *s = g_stream; return 0; }
int rocblas_set_stream(void* handle, void* s) { g_stream = s; return 0; }
int rocblas_get_pointer_mode(void* handle, int* mode) { *mode = 0; return 0; }
int rocblas_gemm_ex(void* h, int ta, int tb, int m, int n, int k, const void* alpha, const void* a, int a_type,
                    int lda, const void* b, int b_type, int ldb, const void* beta, const void* c, int c_type,
                    int ldc, void* d, int d_type, int ldd, int compute_type, int algo, int32_t solution_index,
                    uint32_t flags) {
    rec("rocblas_gemm_ex", ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, d, ldd, 1);
    return 0;
}
#endif
