// epilogue.hpp — optional epilogue inputs shared by every GEMM kernel.
//
//   C = alpha * acc + beta * Cin + bias[n]
// computed in fp32 and rounded once to the output type.
//  * Cin is the matrix beta scales.  The BLAS form is in place (Cin == C);
//    hipBLASLt and rocBLAS take a separate C and D, which the launchers pass
//    as Cin and C.  Cin has the output's element type and is read only when
//    beta != 0 (so a NaN in it never reaches a beta == 0 result).
//  * bias, when not null, holds one value per column n of the row-major C,
//    i.e. per row of the column-major hipBLAS / hipBLASLt D: hipBLASLt's
//    HIPBLASLT_EPILOGUE_BIAS (a vector of D's row count broadcast over its
//    columns, added after alpha / beta and before the final rounding).  It
//    is shared by every batch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vkb {

struct EpiParams {
    const void* cin;     // never null in a launch (the launcher sets C for in place)
    int64_t ldcin;
    int64_t scin;        // batch stride of Cin (elements)
    const void* bias;    // null: no bias
    int bias_type;       // element type of bias: 0 fp32, 1 fp16, 2 bf16
};

__device__ __forceinline__ float bias_at(const EpiParams& e, int64_t n) {
    if (e.bias_type == 1) return (float)((const _Float16*)e.bias)[n];
    if (e.bias_type == 2) return (float)((const __bf16*)e.bias)[n];
    return ((const float*)e.bias)[n];
}

// bias of four consecutive columns n .. n + 3 (valid ones only), added to x
__device__ __forceinline__ void add_bias4(const EpiParams& e, int64_t n, int nvalid, float* x) {
    if (!e.bias) return;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (i < nvalid) x[i] += bias_at(e, n + i);
}

}  // namespace vkb
