/*
 * vkblas_hipblas.h — the hipBLAS ABI exported by libvkblas_hipblas.so.
 *
 * The library is an LD_PRELOAD / dlopen drop-in for the real hipBLAS, as the
 * reference's src/vkblas_hipblas.c is.  Signatures are hipBLAS 3.x ones
 * (ROCm 7.2); the shim includes this header next to <hipblas/hipblas.h>, so
 * the compiler checks every declaration here against the vendor's.
 *
 * Computed by this library (gfx950 kernels): Sgemm*, Hgemm*, and GemmEx* (plain,
 * strided-batched and pointer-array batched) with
 * fp32 data, fp16 data (fp16 or fp32 result) and bf16 data (bf16 or fp32
 * result).  Forwarded to the real hipBLAS when declined (degenerate sizes,
 * other types).
 */
#pragma once
#include <hipblas/hipblas.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference src/vkblas_hipblas.c:403-408 */
hipblasStatus_t hipblasSgemm(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                             int m, int n, int k, const float* alpha, const float* AP, int lda,
                             const float* BP, int ldb, const float* beta, float* CP, int ldc);
/* reference src/vkblas_hipblas.c:409-416 */
hipblasStatus_t hipblasSgemmStridedBatched(hipblasHandle_t handle, hipblasOperation_t transA,
                                           hipblasOperation_t transB, int m, int n, int k, const float* alpha,
                                           const float* AP, int lda, long long strideA, const float* BP,
                                           int ldb, long long strideB, const float* beta, float* CP, int ldc,
                                           long long strideC, int batchCount);
/* reference src/vkblas_hipblas.c:454-466 (hipBLAS >= 3 signature, lines 19-35) */
hipblasStatus_t hipblasGemmEx(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                              int m, int n, int k, const void* alpha, const void* A, hipDataType aType, int lda,
                              const void* B, hipDataType bType, int ldb, const void* beta, void* C,
                              hipDataType cType, int ldc, hipblasComputeType_t computeType,
                              hipblasGemmAlgo_t algo);
/* reference src/vkblas_hipblas.c:417-432 (hipBLAS 2 name; same as hipblasGemmEx) */
hipblasStatus_t hipblasGemmEx_v2(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                 int m, int n, int k, const void* alpha, const void* A, hipDataType aType,
                                 int lda, const void* B, hipDataType bType, int ldb, const void* beta, void* C,
                                 hipDataType cType, int ldc, hipblasComputeType_t computeType,
                                 hipblasGemmAlgo_t algo);
/* reference src/vkblas_hipblas.c:433-453 (hipBLAS 2 name) */
hipblasStatus_t hipblasGemmStridedBatchedEx_v2(hipblasHandle_t handle, hipblasOperation_t transA,
                                               hipblasOperation_t transB, int m, int n, int k,
                                               const void* alpha, const void* A, hipDataType aType, int lda,
                                               hipblasStride strideA, const void* B, hipDataType bType,
                                               int ldb, hipblasStride strideB, const void* beta, void* C,
                                               hipDataType cType, int ldc, hipblasStride strideC,
                                               int batchCount, hipblasComputeType_t computeType,
                                               hipblasGemmAlgo_t algo);
/* New relative to the reference (north star): unsuffixed strided Ex, Hgemm
 * family, and the 64-bit-size variants of each. */
hipblasStatus_t hipblasGemmStridedBatchedEx(hipblasHandle_t handle, hipblasOperation_t transA,
                                            hipblasOperation_t transB, int m, int n, int k, const void* alpha,
                                            const void* A, hipDataType aType, int lda, hipblasStride strideA,
                                            const void* B, hipDataType bType, int ldb, hipblasStride strideB,
                                            const void* beta, void* C, hipDataType cType, int ldc,
                                            hipblasStride strideC, int batchCount,
                                            hipblasComputeType_t computeType, hipblasGemmAlgo_t algo);
hipblasStatus_t hipblasHgemm(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                             int m, int n, int k, const hipblasHalf* alpha, const hipblasHalf* AP, int lda,
                             const hipblasHalf* BP, int ldb, const hipblasHalf* beta, hipblasHalf* CP, int ldc);
hipblasStatus_t hipblasHgemmStridedBatched(hipblasHandle_t handle, hipblasOperation_t transA,
                                           hipblasOperation_t transB, int m, int n, int k,
                                           const hipblasHalf* alpha, const hipblasHalf* AP, int lda,
                                           long long strideA, const hipblasHalf* BP, int ldb, long long strideB,
                                           const hipblasHalf* beta, hipblasHalf* CP, int ldc, long long strideC,
                                           int batchCount);
hipblasStatus_t hipblasSgemm_64(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                int64_t m, int64_t n, int64_t k, const float* alpha, const float* AP,
                                int64_t lda, const float* BP, int64_t ldb, const float* beta, float* CP,
                                int64_t ldc);
hipblasStatus_t hipblasSgemmStridedBatched_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                              hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                              const float* alpha, const float* AP, int64_t lda,
                                              long long strideA, const float* BP, int64_t ldb,
                                              long long strideB, const float* beta, float* CP, int64_t ldc,
                                              long long strideC, int64_t batchCount);
hipblasStatus_t hipblasHgemm_64(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                int64_t m, int64_t n, int64_t k, const hipblasHalf* alpha,
                                const hipblasHalf* AP, int64_t lda, const hipblasHalf* BP, int64_t ldb,
                                const hipblasHalf* beta, hipblasHalf* CP, int64_t ldc);
hipblasStatus_t hipblasHgemmStridedBatched_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                              hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                              const hipblasHalf* alpha, const hipblasHalf* AP, int64_t lda,
                                              long long strideA, const hipblasHalf* BP, int64_t ldb,
                                              long long strideB, const hipblasHalf* beta, hipblasHalf* CP,
                                              int64_t ldc, long long strideC, int64_t batchCount);
hipblasStatus_t hipblasGemmEx_64(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                 int64_t m, int64_t n, int64_t k, const void* alpha, const void* A,
                                 hipDataType aType, int64_t lda, const void* B, hipDataType bType, int64_t ldb,
                                 const void* beta, void* C, hipDataType cType, int64_t ldc,
                                 hipblasComputeType_t computeType, hipblasGemmAlgo_t algo);
hipblasStatus_t hipblasGemmStridedBatchedEx_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                               hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                               const void* alpha, const void* A, hipDataType aType,
                                               int64_t lda, hipblasStride strideA, const void* B,
                                               hipDataType bType, int64_t ldb, hipblasStride strideB,
                                               const void* beta, void* C, hipDataType cType, int64_t ldc,
                                               hipblasStride strideC, int64_t batchCount,
                                               hipblasComputeType_t computeType, hipblasGemmAlgo_t algo);

/* Handle / state, forwarded (reference src/vkblas_hipblas.c:69-123).  The
 * handle is the real hipBLAS handle; stream and pointer mode are per handle. */
hipblasStatus_t hipblasCreate(hipblasHandle_t* handle);
hipblasStatus_t hipblasDestroy(hipblasHandle_t handle);
hipblasStatus_t hipblasSetStream(hipblasHandle_t handle, hipStream_t streamId);
hipblasStatus_t hipblasGetStream(hipblasHandle_t handle, hipStream_t* streamId);
hipblasStatus_t hipblasSetPointerMode(hipblasHandle_t handle, hipblasPointerMode_t mode);
hipblasStatus_t hipblasGetPointerMode(hipblasHandle_t handle, hipblasPointerMode_t* mode);
hipblasStatus_t hipblasSetAtomicsMode(hipblasHandle_t handle, hipblasAtomicsMode_t atomics_mode);
hipblasStatus_t hipblasSetWorkspace(hipblasHandle_t handle, void* workspace, size_t workspaceSizeInBytes);
hipblasStatus_t hipblasGetVersion(hipblasHandle_t handle, int* version);
const char* hipblasStatusToString(hipblasStatus_t status);

/* Forward-only GEMMs (reference src/vkblas_hipblas.c:467-630; this build
 * forwards them instead of running an fp64 / complex engine). */
hipblasStatus_t hipblasDgemm(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                             int m, int n, int k, const double* alpha, const double* AP, int lda,
                             const double* BP, int ldb, const double* beta, double* CP, int ldc);
hipblasStatus_t hipblasDgemmStridedBatched(hipblasHandle_t handle, hipblasOperation_t transA,
                                           hipblasOperation_t transB, int m, int n, int k, const double* alpha,
                                           const double* AP, int lda, long long strideA, const double* BP,
                                           int ldb, long long strideB, const double* beta, double* CP, int ldc,
                                           long long strideC, int batchCount);
hipblasStatus_t hipblasCgemm(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                             int m, int n, int k, const hipComplex* alpha, const hipComplex* AP, int lda,
                             const hipComplex* BP, int ldb, const hipComplex* beta, hipComplex* CP, int ldc);
hipblasStatus_t hipblasCgemm_v2(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                int m, int n, int k, const hipComplex* alpha, const hipComplex* AP, int lda,
                                const hipComplex* BP, int ldb, const hipComplex* beta, hipComplex* CP, int ldc);
hipblasStatus_t hipblasZgemm(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                             int m, int n, int k, const hipDoubleComplex* alpha, const hipDoubleComplex* AP,
                             int lda, const hipDoubleComplex* BP, int ldb, const hipDoubleComplex* beta,
                             hipDoubleComplex* CP, int ldc);
hipblasStatus_t hipblasZgemm_v2(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                int m, int n, int k, const hipDoubleComplex* alpha, const hipDoubleComplex* AP,
                                int lda, const hipDoubleComplex* BP, int ldb, const hipDoubleComplex* beta,
                                hipDoubleComplex* CP, int ldc);
hipblasStatus_t hipblasCgemmStridedBatched(hipblasHandle_t handle, hipblasOperation_t transA,
                                           hipblasOperation_t transB, int m, int n, int k,
                                           const hipComplex* alpha, const hipComplex* AP, int lda,
                                           long long strideA, const hipComplex* BP, int ldb, long long strideB,
                                           const hipComplex* beta, hipComplex* CP, int ldc, long long strideC,
                                           int batchCount);
hipblasStatus_t hipblasCgemmStridedBatched_v2(hipblasHandle_t handle, hipblasOperation_t transA,
                                              hipblasOperation_t transB, int m, int n, int k,
                                              const hipComplex* alpha, const hipComplex* AP, int lda,
                                              long long strideA, const hipComplex* BP, int ldb,
                                              long long strideB, const hipComplex* beta, hipComplex* CP,
                                              int ldc, long long strideC, int batchCount);
hipblasStatus_t hipblasZgemmStridedBatched(hipblasHandle_t handle, hipblasOperation_t transA,
                                           hipblasOperation_t transB, int m, int n, int k,
                                           const hipDoubleComplex* alpha, const hipDoubleComplex* AP, int lda,
                                           long long strideA, const hipDoubleComplex* BP, int ldb,
                                           long long strideB, const hipDoubleComplex* beta,
                                           hipDoubleComplex* CP, int ldc, long long strideC, int batchCount);
hipblasStatus_t hipblasZgemmStridedBatched_v2(hipblasHandle_t handle, hipblasOperation_t transA,
                                              hipblasOperation_t transB, int m, int n, int k,
                                              const hipDoubleComplex* alpha, const hipDoubleComplex* AP,
                                              int lda, long long strideA, const hipDoubleComplex* BP, int ldb,
                                              long long strideB, const hipDoubleComplex* beta,
                                              hipDoubleComplex* CP, int ldc, long long strideC, int batchCount);

/* Pure forwarders (reference src/vkblas_hipblas.c:632-800).  hipBLAS 3 has
 * no _v2 names; each _v2 export calls the unsuffixed real symbol. */
hipblasStatus_t hipblasSdot(hipblasHandle_t h, int n, const float* x, int incx, const float* y, int incy,
                            float* result);
hipblasStatus_t hipblasDdot(hipblasHandle_t h, int n, const double* x, int incx, const double* y, int incy,
                            double* result);
hipblasStatus_t hipblasCdotc(hipblasHandle_t h, int n, const hipComplex* x, int incx, const hipComplex* y,
                             int incy, hipComplex* result);
hipblasStatus_t hipblasCdotc_v2(hipblasHandle_t h, int n, const hipComplex* x, int incx, const hipComplex* y,
                                int incy, hipComplex* result);
hipblasStatus_t hipblasCdotu(hipblasHandle_t h, int n, const hipComplex* x, int incx, const hipComplex* y,
                             int incy, hipComplex* result);
hipblasStatus_t hipblasCdotu_v2(hipblasHandle_t h, int n, const hipComplex* x, int incx, const hipComplex* y,
                                int incy, hipComplex* result);
hipblasStatus_t hipblasZdotc(hipblasHandle_t h, int n, const hipDoubleComplex* x, int incx,
                             const hipDoubleComplex* y, int incy, hipDoubleComplex* result);
hipblasStatus_t hipblasZdotc_v2(hipblasHandle_t h, int n, const hipDoubleComplex* x, int incx,
                                const hipDoubleComplex* y, int incy, hipDoubleComplex* result);
hipblasStatus_t hipblasZdotu(hipblasHandle_t h, int n, const hipDoubleComplex* x, int incx,
                             const hipDoubleComplex* y, int incy, hipDoubleComplex* result);
hipblasStatus_t hipblasZdotu_v2(hipblasHandle_t h, int n, const hipDoubleComplex* x, int incx,
                                const hipDoubleComplex* y, int incy, hipDoubleComplex* result);
hipblasStatus_t hipblasDotEx(hipblasHandle_t h, int n, const void* x, hipDataType xType, int incx,
                             const void* y, hipDataType yType, int incy, void* result, hipDataType resultType,
                             hipDataType executionType);
hipblasStatus_t hipblasDotEx_v2(hipblasHandle_t h, int n, const void* x, hipDataType xType, int incx,
                                const void* y, hipDataType yType, int incy, void* result,
                                hipDataType resultType, hipDataType executionType);
hipblasStatus_t hipblasSgemv(hipblasHandle_t h, hipblasOperation_t trans, int m, int n, const float* alpha,
                             const float* AP, int lda, const float* x, int incx, const float* beta, float* y,
                             int incy);
hipblasStatus_t hipblasDgemv(hipblasHandle_t h, hipblasOperation_t trans, int m, int n, const double* alpha,
                             const double* AP, int lda, const double* x, int incx, const double* beta, double* y,
                             int incy);
hipblasStatus_t hipblasCgemv(hipblasHandle_t h, hipblasOperation_t trans, int m, int n, const hipComplex* alpha,
                             const hipComplex* AP, int lda, const hipComplex* x, int incx,
                             const hipComplex* beta, hipComplex* y, int incy);
hipblasStatus_t hipblasCgemv_v2(hipblasHandle_t h, hipblasOperation_t trans, int m, int n,
                                const hipComplex* alpha, const hipComplex* AP, int lda, const hipComplex* x,
                                int incx, const hipComplex* beta, hipComplex* y, int incy);
hipblasStatus_t hipblasZgemv(hipblasHandle_t h, hipblasOperation_t trans, int m, int n,
                             const hipDoubleComplex* alpha, const hipDoubleComplex* AP, int lda,
                             const hipDoubleComplex* x, int incx, const hipDoubleComplex* beta,
                             hipDoubleComplex* y, int incy);
hipblasStatus_t hipblasZgemv_v2(hipblasHandle_t h, hipblasOperation_t trans, int m, int n,
                                const hipDoubleComplex* alpha, const hipDoubleComplex* AP, int lda,
                                const hipDoubleComplex* x, int incx, const hipDoubleComplex* beta,
                                hipDoubleComplex* y, int incy);
#define VKBLAS_TRSM_DECL(name, T)                                                                      \
    hipblasStatus_t name(hipblasHandle_t h, hipblasSideMode_t side, hipblasFillMode_t uplo,            \
                         hipblasOperation_t transA, hipblasDiagType_t diag, int m, int n, const T* alpha, \
                         const T* AP, int lda, T* BP, int ldb);
#define VKBLAS_TRSMB_DECL(name, T)                                                                     \
    hipblasStatus_t name(hipblasHandle_t h, hipblasSideMode_t side, hipblasFillMode_t uplo,            \
                         hipblasOperation_t transA, hipblasDiagType_t diag, int m, int n, const T* alpha, \
                         const T* const AP[], int lda, T* const BP[], int ldb, int batchCount);
#define VKBLAS_GELS_DECL(name, T)                                                                      \
    hipblasStatus_t name(hipblasHandle_t h, hipblasOperation_t trans, const int m, const int n,        \
                         const int nrhs, T* const A[], const int lda, T* const B[], const int ldb,      \
                         int* info, int* deviceInfo, const int batchCount);
#define VKBLAS_GEQRF_DECL(name, T)                                                                     \
    hipblasStatus_t name(hipblasHandle_t h, const int m, const int n, T* const A[], const int lda,     \
                         T* const ipiv[], int* info, const int batchCount);
#define VKBLAS_GETRF_DECL(name, T)                                                                     \
    hipblasStatus_t name(hipblasHandle_t h, const int n, T* const A[], const int lda, int* ipiv,       \
                         int* info, const int batchCount);
#define VKBLAS_GETRS_DECL(name, T)                                                                     \
    hipblasStatus_t name(hipblasHandle_t h, const hipblasOperation_t trans, const int n,               \
                         const int nrhs, T* const A[], const int lda, const int* ipiv, T* const B[],    \
                         const int ldb, int* info, const int batchCount);
#define VKBLAS_FOUR(DECL, S, D, C, Z)                                                                  \
    DECL(hipblas##S, float) DECL(hipblas##D, double) DECL(hipblas##C, hipComplex)                      \
    DECL(hipblas##C##_v2, hipComplex) DECL(hipblas##Z, hipDoubleComplex)                               \
    DECL(hipblas##Z##_v2, hipDoubleComplex)
VKBLAS_FOUR(VKBLAS_TRSM_DECL, Strsm, Dtrsm, Ctrsm, Ztrsm)
VKBLAS_FOUR(VKBLAS_TRSMB_DECL, StrsmBatched, DtrsmBatched, CtrsmBatched, ZtrsmBatched)
VKBLAS_FOUR(VKBLAS_GELS_DECL, SgelsBatched, DgelsBatched, CgelsBatched, ZgelsBatched)
VKBLAS_FOUR(VKBLAS_GEQRF_DECL, SgeqrfBatched, DgeqrfBatched, CgeqrfBatched, ZgeqrfBatched)
VKBLAS_FOUR(VKBLAS_GETRF_DECL, SgetrfBatched, DgetrfBatched, CgetrfBatched, ZgetrfBatched)
VKBLAS_FOUR(VKBLAS_GETRS_DECL, SgetrsBatched, DgetrsBatched, CgetrsBatched, ZgetrsBatched)

/* Pointer-array batched GEMMs: no counterpart in the reference, which left
 * them to the real hipBLAS.  A, B, C are device arrays of batchCount matrix
 * pointers; computed for the same types as the non-batched entries. */
hipblasStatus_t hipblasSgemmBatched(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                    int m, int n, int k, const float* alpha, const float* const AP[], int lda,
                                    const float* const BP[], int ldb, const float* beta, float* const CP[], int ldc,
                                    int batchCount);
hipblasStatus_t hipblasSgemmBatched_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                       hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                       const float* alpha, const float* const AP[], int64_t lda,
                                       const float* const BP[], int64_t ldb, const float* beta, float* const CP[],
                                       int64_t ldc, int64_t batchCount);
hipblasStatus_t hipblasHgemmBatched(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                    int m, int n, int k, const hipblasHalf* alpha, const hipblasHalf* const AP[],
                                    int lda, const hipblasHalf* const BP[], int ldb, const hipblasHalf* beta,
                                    hipblasHalf* const CP[], int ldc, int batchCount);
hipblasStatus_t hipblasHgemmBatched_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                       hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                       const hipblasHalf* alpha, const hipblasHalf* const AP[], int64_t lda,
                                       const hipblasHalf* const BP[], int64_t ldb, const hipblasHalf* beta,
                                       hipblasHalf* const CP[], int64_t ldc, int64_t batchCount);
hipblasStatus_t hipblasGemmBatchedEx(hipblasHandle_t handle, hipblasOperation_t transA, hipblasOperation_t transB,
                                     int m, int n, int k, const void* alpha, const void* A[], hipDataType aType,
                                     int lda, const void* B[], hipDataType bType, int ldb, const void* beta,
                                     void* C[], hipDataType cType, int ldc, int batchCount,
                                     hipblasComputeType_t computeType, hipblasGemmAlgo_t algo);
hipblasStatus_t hipblasGemmBatchedEx_64(hipblasHandle_t handle, hipblasOperation_t transA,
                                        hipblasOperation_t transB, int64_t m, int64_t n, int64_t k,
                                        const void* alpha, const void* A[], hipDataType aType, int64_t lda,
                                        const void* B[], hipDataType bType, int64_t ldb, const void* beta,
                                        void* C[], hipDataType cType, int64_t ldc, int64_t batchCount,
                                        hipblasComputeType_t computeType, hipblasGemmAlgo_t algo);

#ifdef __cplusplus
}
#endif
