// gemm_f16s.hip — fp16 inputs, fp32 output (hipblasGemmEx 16F/16F/32F), and
// fp32 split-K partials of fp16 GEMMs.  No counterpart kernel in the
// reference, which forwarded this type combination to the vendor library
// (src/vkblas_hipblas.c:428-431).
#include "gemm_launch.hpp"

extern "C" int vkb_launch_gemm_f16s_impl(const vkb_gemm_args* a, int tile, void* stream) {
    return vkb::launch_gemm_typed<_Float16, float>(a, tile, (hipStream_t)stream);
}
