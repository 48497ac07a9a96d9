/*
 * vkblas_rocblas.h — the rocBLAS entry points exported by libvkblas_hipblas.so.
 *
 * PyTorch-ROCm's hipBLAS backend computes fp16 / bf16 GEMMs by calling
 * rocblas_gemm_ex / rocblas_gemm_strided_batched_ex on the handle directly
 * (a hipBLAS handle is a rocBLAS handle on AMD), bypassing the hipBLAS symbols,
 * so an LD_PRELOAD drop-in has to interpose this layer too, as the reference
 * does (src/vkblas_hipblas.c:802-955).  Signatures are rocBLAS 5.x (ROCm 7.2);
 * the shim includes this header after <rocblas/rocblas.h>, so the compiler
 * checks every declaration against the vendor's.  The names are parenthesised
 * because rocblas.h also defines function-like macros of the same names.
 *
 * Computed by this library: fp32 x fp32 -> fp32, fp16 x fp16 -> fp16,
 * fp16 x fp16 -> fp32, bf16 x bf16 -> bf16 and bf16 x bf16 -> fp32 with
 * compute type f32_r; any D (D == C, or a separate D
 * that C is copied into first when beta may be nonzero).  Everything else
 * (other types, other compute types, solution queries, degenerate sizes) is
 * forwarded to the real rocBLAS of the process.
 */
#pragma once
#include <rocblas/rocblas.h>

#ifdef __cplusplus
extern "C" {
#endif

/* reference src/vkblas_hipblas.c:824-887 */
rocblas_status(rocblas_gemm_ex)(rocblas_handle handle, rocblas_operation transA, rocblas_operation transB,
                                rocblas_int m, rocblas_int n, rocblas_int k, const void* alpha, const void* a,
                                rocblas_datatype a_type, rocblas_int lda, const void* b, rocblas_datatype b_type,
                                rocblas_int ldb, const void* beta, const void* c, rocblas_datatype c_type,
                                rocblas_int ldc, void* d, rocblas_datatype d_type, rocblas_int ldd,
                                rocblas_datatype compute_type, rocblas_gemm_algo algo, int32_t solution_index,
                                uint32_t flags);

/* reference src/vkblas_hipblas.c:889-955 */
rocblas_status(rocblas_gemm_strided_batched_ex)(
    rocblas_handle handle, rocblas_operation transA, rocblas_operation transB, rocblas_int m, rocblas_int n,
    rocblas_int k, const void* alpha, const void* a, rocblas_datatype a_type, rocblas_int lda,
    rocblas_stride stride_a, const void* b, rocblas_datatype b_type, rocblas_int ldb, rocblas_stride stride_b,
    const void* beta, const void* c, rocblas_datatype c_type, rocblas_int ldc, rocblas_stride stride_c, void* d,
    rocblas_datatype d_type, rocblas_int ldd, rocblas_stride stride_d, rocblas_int batch_count,
    rocblas_datatype compute_type, rocblas_gemm_algo algo, int32_t solution_index, uint32_t flags);

/* 64-bit-integer variants (no reference counterpart; same semantics) */
rocblas_status(rocblas_gemm_ex_64)(rocblas_handle handle, rocblas_operation transA, rocblas_operation transB,
                                   int64_t m, int64_t n, int64_t k, const void* alpha, const void* a,
                                   rocblas_datatype a_type, int64_t lda, const void* b, rocblas_datatype b_type,
                                   int64_t ldb, const void* beta, const void* c, rocblas_datatype c_type,
                                   int64_t ldc, void* d, rocblas_datatype d_type, int64_t ldd,
                                   rocblas_datatype compute_type, rocblas_gemm_algo algo, int32_t solution_index,
                                   uint32_t flags);

rocblas_status(rocblas_gemm_strided_batched_ex_64)(
    rocblas_handle handle, rocblas_operation transA, rocblas_operation transB, int64_t m, int64_t n, int64_t k,
    const void* alpha, const void* a, rocblas_datatype a_type, int64_t lda, rocblas_stride stride_a,
    const void* b, rocblas_datatype b_type, int64_t ldb, rocblas_stride stride_b, const void* beta,
    const void* c, rocblas_datatype c_type, int64_t ldc, rocblas_stride stride_c, void* d,
    rocblas_datatype d_type, int64_t ldd, rocblas_stride stride_d, int64_t batch_count,
    rocblas_datatype compute_type, rocblas_gemm_algo algo, int32_t solution_index, uint32_t flags);

/* Pointer-array batched: no counterpart in the reference, which forwarded it.
 * a, b, c, d are device arrays of batch_count matrix pointers; D must be C. */
rocblas_status(rocblas_gemm_batched_ex)(rocblas_handle handle, rocblas_operation transA, rocblas_operation transB,
                                        rocblas_int m, rocblas_int n, rocblas_int k, const void* alpha,
                                        const void* a, rocblas_datatype a_type, rocblas_int lda, const void* b,
                                        rocblas_datatype b_type, rocblas_int ldb, const void* beta, const void* c,
                                        rocblas_datatype c_type, rocblas_int ldc, void* d, rocblas_datatype d_type,
                                        rocblas_int ldd, rocblas_int batch_count, rocblas_datatype compute_type,
                                        rocblas_gemm_algo algo, int32_t solution_index, uint32_t flags);
rocblas_status(rocblas_gemm_batched_ex_64)(rocblas_handle handle, rocblas_operation transA,
                                           rocblas_operation transB, int64_t m, int64_t n, int64_t k,
                                           const void* alpha, const void* a, rocblas_datatype a_type, int64_t lda,
                                           const void* b, rocblas_datatype b_type, int64_t ldb, const void* beta,
                                           const void* c, rocblas_datatype c_type, int64_t ldc, void* d,
                                           rocblas_datatype d_type, int64_t ldd, int64_t batch_count,
                                           rocblas_datatype compute_type, rocblas_gemm_algo algo,
                                           int32_t solution_index, uint32_t flags);

#ifdef __cplusplus
}
#endif
