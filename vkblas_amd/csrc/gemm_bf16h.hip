// gemm_bf16h.hip — bf16 GEMM, bf16 output: vkblas_gemm_bf16 / _bf16_hipblas and
// hipblasGemmEx / rocblas_gemm_ex with 16BF inputs and output.  Replaces the
// reference's HALF_TYPE = 2 instantiations of its half-precision shaders
// (src/shaders/gemm_half_128x128_bankfree_tmpl.comp:26-47, dispatched from
// src/vkblas.c:3345-3512): bf16 operands, fp32 MFMA accumulation
// (v_mfma_f32_*_bf16), one round-to-nearest-even to bf16.
#include "gemm_launch.hpp"

extern "C" int vkb_launch_gemm_bf16h_impl(const vkb_gemm_args* a, int tile, void* stream) {
    return vkb::launch_gemm_typed<__bf16, __bf16>(a, tile, (hipStream_t)stream);
}
