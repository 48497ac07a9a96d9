// gemm_f32h.hip — fp32 inputs, fp16 output (hipblasGemmEx 32F/32F/16F with
// fp32 compute): fp32 MFMA accumulation, one RNE rounding to fp16 in the
// epilogue.  No counterpart kernel in the reference, which forwarded every
// mixed fp32 / 16-bit Ex combination to the vendor library
// (src/vkblas_hipblas.c:428-431).
#include "gemm_launch.hpp"

extern "C" int vkb_launch_gemm_f32h_impl(const vkb_gemm_args* a, int tile, void* stream) {
    return vkb::launch_gemm_typed<float, _Float16>(a, tile, (hipStream_t)stream);
}
