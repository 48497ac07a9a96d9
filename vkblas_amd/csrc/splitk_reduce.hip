// splitk_reduce.hip — split-K pass 2 and the GEMM launch dispatcher.
//
// Pass 2 replaces the reference's splitk_reduce_f32.comp / splitk_reduce_hgemm.comp
// (reduce loop src/shaders/splitk_reduce_f32.comp:15-24): every output sums its
// fp32 partials in the fixed order s = 0 .. split-1, then applies alpha / beta
// and rounds once to the output type (fp32, fp16 or bf16).  No atomics, so results are bitwise
// reproducible run to run.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "vkb_launch.h"

extern "C" int vkb_launch_gemm_f32_impl(const vkb_gemm_args* a, int tile, void* stream);
extern "C" int vkb_launch_gemm_f16h_impl(const vkb_gemm_args* a, int tile, void* stream);
extern "C" int vkb_launch_gemm_f16s_impl(const vkb_gemm_args* a, int tile, void* stream);
extern "C" int vkb_launch_gemm_bf16h_impl(const vkb_gemm_args* a, int tile, void* stream);
extern "C" int vkb_launch_gemm_bf16s_impl(const vkb_gemm_args* a, int tile, void* stream);

namespace {

template <typename TC>
__device__ __forceinline__ void put(TC* p, float v) { *p = (TC)v; }

// One thread per 4 consecutive n of one row.  Partials of 8 splits are in
// flight per iteration; the additions still run in split order.
template <typename TC>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(
    const float* __restrict__ P, int64_t ss, uint32_t split, uint32_t M, uint32_t N,
    TC* __restrict__ C, int64_t ldc, float alpha, float beta, int mode,
    const void* alpha_dev, const void* beta_dev) {
    const uint32_t ng = (N + 3) >> 2;
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)M * ng) return;
    const uint32_t m = (uint32_t)(idx / ng);
    const uint32_t n = (uint32_t)(idx - (uint64_t)m * ng) * 4;
    const bool vec = (N & 3u) == 0 && (ss & 3) == 0;
    const int nv = (int)min(4u, N - n);
    if (mode == 1) {
        alpha = *(const float*)alpha_dev;
        beta = *(const float*)beta_dev;
    } else if (mode == 2) {
        alpha = (float)*(const _Float16*)alpha_dev;
        beta = (float)*(const _Float16*)beta_dev;
    }
    const float* src = P + (uint64_t)m * N + n;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    uint32_t s = 0;
    if (vec) {
        for (; s + 8 <= split; s += 8) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = *(const float4*)(src + (int64_t)(s + u) * ss);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc[0] += v[u].x; acc[1] += v[u].y; acc[2] += v[u].z; acc[3] += v[u].w;
            }
        }
        for (; s < split; ++s) {
            const float4 v = *(const float4*)(src + (int64_t)s * ss);
            acc[0] += v.x; acc[1] += v.y; acc[2] += v.z; acc[3] += v.w;
        }
    } else {
        for (; s < split; ++s) {
            const float* q = src + (int64_t)s * ss;
            for (int e = 0; e < nv; ++e) acc[e] += q[e];
        }
    }
    TC* dst = C + (int64_t)m * ldc + n;
    for (int e = 0; e < nv; ++e) {
        float y = alpha * acc[e];
        if (beta != 0.0f) y += beta * (float)dst[e];
        put<TC>(dst + e, y);
    }
}

}  // namespace

extern "C" int vkb_launch_splitk_reduce(const float* P, int64_t stride_split, uint32_t split,
                                        uint32_t M, uint32_t N, void* C, int64_t ldc, int c_type,
                                        float alpha, float beta, int scalar_mode,
                                        const void* alpha_dev, const void* beta_dev, void* stream) {
    const uint64_t groups = (uint64_t)M * ((N + 3) / 4);
    const uint64_t blocks = (groups + 255) / 256;
    if (blocks == 0 || blocks > 0x7fffffffull || split == 0) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    if (c_type == VKB_T_F32) {
        hipLaunchKernelGGL(splitk_reduce_kernel<float>, dim3((uint32_t)blocks), dim3(256), 0, st, P,
                           stride_split, split, M, N, (float*)C, ldc, alpha, beta, scalar_mode,
                           alpha_dev, beta_dev);
    } else if (c_type == VKB_T_F16) {
        hipLaunchKernelGGL(splitk_reduce_kernel<_Float16>, dim3((uint32_t)blocks), dim3(256), 0, st, P,
                           stride_split, split, M, N, (_Float16*)C, ldc, alpha, beta, scalar_mode,
                           alpha_dev, beta_dev);
    } else if (c_type == VKB_T_BF16) {
        hipLaunchKernelGGL(splitk_reduce_kernel<__bf16>, dim3((uint32_t)blocks), dim3(256), 0, st, P,
                           stride_split, split, M, N, (__bf16*)C, ldc, alpha, beta, scalar_mode,
                           alpha_dev, beta_dev);
    } else {
        return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

extern "C" uint32_t vkb_tile_bm(int tile) {
    return tile == VKB_TILE_256 ? 256u : tile == VKB_TILE_128 ? 128u : 64u;
}
extern "C" uint32_t vkb_tile_bn(int tile) { return vkb_tile_bm(tile); }
extern "C" uint32_t vkb_tile_bk(int ab_type) { return ab_type == VKB_T_F32 ? 32u : 64u; }

extern "C" int vkb_launch_gemm(const vkb_gemm_args* a, int tile, void* stream) {
    if (a->ab_type == VKB_T_F32 && a->c_type == VKB_T_F32) return vkb_launch_gemm_f32_impl(a, tile, stream);
    if (a->ab_type == VKB_T_F16 && a->c_type == VKB_T_F16) return vkb_launch_gemm_f16h_impl(a, tile, stream);
    if (a->ab_type == VKB_T_F16 && a->c_type == VKB_T_F32) return vkb_launch_gemm_f16s_impl(a, tile, stream);
    if (a->ab_type == VKB_T_BF16 && a->c_type == VKB_T_BF16) return vkb_launch_gemm_bf16h_impl(a, tile, stream);
    if (a->ab_type == VKB_T_BF16 && a->c_type == VKB_T_F32) return vkb_launch_gemm_bf16s_impl(a, tile, stream);
    return (int)hipErrorInvalidValue;
}
