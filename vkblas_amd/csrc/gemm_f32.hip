// gemm_f32.hip — fp32 GEMM instantiations (v_mfma_f32_32x32x2_f32).
// Replaces the reference's fp32 tile kernels gemm_f32_64x64_tmpl.comp and
// gemm_f32_128x128_bankfree_tmpl.comp (src/vkblas.c:1759-1868).
#include "gemm_launch.hpp"

extern "C" int vkb_launch_gemm_f32_impl(const vkb_gemm_args* a, int tile, void* stream) {
    return vkb::launch_gemm_typed<float, float>(a, tile, (hipStream_t)stream);
}
