// gemm_f32b.hip — fp32 inputs, bf16 output (hipblasGemmEx 32F/32F/16BF with
// fp32 compute): fp32 MFMA accumulation, one RNE rounding to bf16 in the
// epilogue.  No counterpart kernel in the reference (it forwarded mixed
// Ex combinations, src/vkblas_hipblas.c:428-431).
#include "gemm_launch.hpp"

extern "C" int vkb_launch_gemm_f32b_impl(const vkb_gemm_args* a, int tile, void* stream) {
    return vkb::launch_gemm_typed<float, __bf16>(a, tile, (hipStream_t)stream);
}
