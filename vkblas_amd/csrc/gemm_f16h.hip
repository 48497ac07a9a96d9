// gemm_f16h.hip — fp16 GEMM, fp16 output (v_mfma_f32_32x32x16_f16, fp32
// accumulate, one RNE rounding to fp16 in the epilogue).  Replaces the
// reference's half tile kernels gemm_half_{64x64,128x128,128x256}_bankfree
// (src/vkblas.c:1191-1313).
#include "gemm_launch.hpp"

extern "C" int vkb_launch_gemm_f16h_impl(const vkb_gemm_args* a, int tile, void* stream) {
    return vkb::launch_gemm_typed<_Float16, _Float16>(a, tile, (hipStream_t)stream);
}
