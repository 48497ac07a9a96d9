// mfma_probe.hip — the v_mfma_f32_16x16x32 rate gfx950 sustains with no
// memory traffic, for a given operand data set.  Not a GEMM: it measures the
// ceiling the 16-bit GEMM kernels are held to when the chip runs at its power
// limit, which depends on the data (random fp16 mantissas toggle more
// multiplier bits than bf16 ones, zeros hardly any).  No counterpart in the
// reference, and not part of libvkblas_hipblas.so: it builds into
// bench_probe/libvkblas_probe.so, which only bench.py and its test load.
//
// Each wave holds eight A and four B 16x16x32 fragments (read once from
// `operands`: fragment f is operands[64 f + lane]) and 32 accumulator tiles,
// and issues `iters` rounds of the 32 independent MFMAs that pair them, the
// issue pattern of the GEMM kernel's inner loop with the fragment loads taken
// out.  The MFMAs are inline assembly on fixed accumulator registers, so the
// loop is MFMAs and a branch only.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <bool BF16>
__global__ __launch_bounds__(256) void mfma_probe_kernel(const u32x4* operands, float* out, int iters) {
    const int lane = threadIdx.x & 63;
    u32x4 a[8], b[4];
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = operands[64 * i + lane];
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = operands[64 * (8 + j) + lane];
    floatx4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (BF16)
                    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc[i][j]) : "v"(a[i]), "v"(b[j]));
                else
                    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc[i][j]) : "v"(a[i]), "v"(b[j]));
            }
    }
    // the compiler does not see the MFMAs' latency: wait out the last ones
    // (at most 18 wait states) before the accumulators are read
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) s += acc[i][j][0] + acc[i][j][1] + acc[i][j][2] + acc[i][j][3];
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace

extern "C" int vkblas_mfma_probe(int bf16, const void* operands, float* out, uint32_t blocks, uint32_t iters,
                                 void* stream) {
    if (!operands || !out || blocks == 0 || blocks > (1u << 20) || iters == 0 || iters > (1u << 24) ||
        ((uintptr_t)operands & 15) || ((uintptr_t)out & 3))
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    if (bf16)
        hipLaunchKernelGGL(mfma_probe_kernel<true>, dim3(blocks), dim3(256), 0, st, (const u32x4*)operands, out,
                           (int)iters);
    else
        hipLaunchKernelGGL(mfma_probe_kernel<false>, dim3(blocks), dim3(256), 0, st, (const u32x4*)operands, out,
                           (int)iters);
    return (int)hipGetLastError();
}
