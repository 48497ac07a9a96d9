// gemm_bf16s.hip — bf16 inputs, fp32 output (hipblasGemmEx / rocblas_gemm_ex
// 16BF/16BF/32F, PyTorch's bf16 GEMMs with fp32 results), and the fp32 split-K
// partials of bf16 GEMMs.  The reference forwarded this combination to the
// vendor library (src/vkblas_hipblas.c:426-461 handles only 16BF -> 16BF).
#include "gemm_launch.hpp"

extern "C" int vkb_launch_gemm_bf16s_impl(const vkb_gemm_args* a, int tile, void* stream) {
    return vkb::launch_gemm_typed<__bf16, float>(a, tile, (hipStream_t)stream);
}
