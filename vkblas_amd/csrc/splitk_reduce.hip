// splitk_reduce.hip — split-K pass 2 and the GEMM launch dispatcher.
//
// Pass 2 replaces the reference's splitk_reduce_f32.comp / splitk_reduce_hgemm.comp
// (reduce loop src/shaders/splitk_reduce_f32.comp:15-24): every output sums its
// fp32 partials in an order fixed by the split count alone (four in-order runs
// over quarters of the slices, then the four run sums in order), then applies
// alpha / beta and rounds once to the output type (fp32, fp16 or bf16).  No
// atomics, so results are bitwise reproducible run to run.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "epilogue.hpp"
#include "vkb_launch.h"

extern "C" int vkb_launch_gemm_f32_impl(const vkb_gemm_args* a, int tile, void* stream);
extern "C" int vkb_launch_gemm_f16h_impl(const vkb_gemm_args* a, int tile, void* stream);
extern "C" int vkb_launch_gemm_f16s_impl(const vkb_gemm_args* a, int tile, void* stream);
extern "C" int vkb_launch_gemm_bf16h_impl(const vkb_gemm_args* a, int tile, void* stream);
extern "C" int vkb_launch_gemm_bf16s_impl(const vkb_gemm_args* a, int tile, void* stream);
extern "C" int vkb_launch_gemm_f32h_impl(const vkb_gemm_args* a, int tile, void* stream);
extern "C" int vkb_launch_gemm_f32b_impl(const vkb_gemm_args* a, int tile, void* stream);

namespace {

template <typename TC>
__device__ __forceinline__ void put(TC* p, float v) { *p = (TC)v; }

// A workgroup owns 64 groups of 4 consecutive n (one lane each) and its four
// waves split the slices: wave w sums slices [w S / 4, (w + 1) S / 4) in
// order, 8 partials in flight per iteration, and wave 0 then adds the other
// waves' sums in wave order.  The summation order is fixed by S alone.
constexpr int RWAVES = 4;

template <typename TC>
__global__ __launch_bounds__(64 * RWAVES) void splitk_reduce_kernel(
    const float* __restrict__ P, int64_t ss, uint32_t split, uint32_t M, uint32_t N,
    TC* __restrict__ C, int64_t ldc, float alpha, float beta, int mode,
    const void* alpha_dev, const void* beta_dev, vkb::EpiParams epi) {
    __shared__ float4 wsum[RWAVES - 1][64];
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t ng = (N + 3) >> 2;
    const uint64_t idx = (uint64_t)blockIdx.x * 64 + lane;
    const bool live = idx < (uint64_t)M * ng;
    const uint32_t m = live ? (uint32_t)(idx / ng) : 0u;
    const uint32_t n = live ? (uint32_t)(idx - (uint64_t)m * ng) * 4 : 0u;
    const bool vec = (N & 3u) == 0 && (ss & 3) == 0;
    const int nv = (int)min(4u, N - n);
    const uint32_t s0 = (uint32_t)((uint64_t)split * w / RWAVES);
    const uint32_t s1 = (uint32_t)((uint64_t)split * (w + 1) / RWAVES);
    const float* src = P + (uint64_t)m * N + n;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    uint32_t s = s0;
    if (!live) {
        s = s1;
    } else if (vec) {
        for (; s + 8 <= s1; s += 8) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = *(const float4*)(src + (int64_t)(s + u) * ss);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc[0] += v[u].x; acc[1] += v[u].y; acc[2] += v[u].z; acc[3] += v[u].w;
            }
        }
        for (; s < s1; ++s) {
            const float4 v = *(const float4*)(src + (int64_t)s * ss);
            acc[0] += v.x; acc[1] += v.y; acc[2] += v.z; acc[3] += v.w;
        }
    } else {
        for (; s < s1; ++s) {
            const float* q = src + (int64_t)s * ss;
            for (int e = 0; e < nv; ++e) acc[e] += q[e];
        }
    }
    if (w > 0) wsum[w - 1][lane] = float4{acc[0], acc[1], acc[2], acc[3]};
    __syncthreads();
    if (w != 0 || !live) return;
#pragma unroll
    for (int g = 0; g < RWAVES - 1; ++g) {
        const float4 v = wsum[g][lane];
        acc[0] += v.x; acc[1] += v.y; acc[2] += v.z; acc[3] += v.w;
    }
    if (mode == 1) {
        alpha = *(const float*)alpha_dev;
        beta = *(const float*)beta_dev;
    } else if (mode == 2) {
        alpha = (float)*(const _Float16*)alpha_dev;
        beta = (float)*(const _Float16*)beta_dev;
    }
    TC* dst = C + (int64_t)m * ldc + n;
    const TC* cin = (const TC*)epi.cin + (int64_t)m * epi.ldcin + n;
    for (int e = 0; e < nv; ++e) {
        float y = alpha * acc[e];
        if (beta != 0.0f) y += beta * (float)cin[e];
        if (epi.bias) y += vkb::bias_at(epi, (int64_t)n + e);
        put<TC>(dst + e, y);
    }
}

}  // namespace

extern "C" int vkb_launch_splitk_reduce(const float* P, int64_t stride_split, uint32_t split,
                                        uint32_t M, uint32_t N, void* C, int64_t ldc, int c_type,
                                        float alpha, float beta, int scalar_mode,
                                        const void* alpha_dev, const void* beta_dev,
                                        const vkb_epilogue_args* ep, void* stream) {
    const uint64_t groups = (uint64_t)M * ((N + 3) / 4);
    const uint64_t blocks = (groups + 63) / 64;
    if (blocks == 0 || blocks > 0x7fffffffull || split == 0) return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    vkb::EpiParams epi;
    epi.cin = ep && ep->c_in ? ep->c_in : C;
    epi.ldcin = ep && ep->c_in ? ep->ldc_in : ldc;
    epi.scin = 0;
    epi.bias = ep ? ep->bias : nullptr;
    epi.bias_type = ep ? ep->bias_type : 0;
    if (c_type == VKB_T_F32) {
        hipLaunchKernelGGL(splitk_reduce_kernel<float>, dim3((uint32_t)blocks), dim3(64 * RWAVES), 0, st, P,
                           stride_split, split, M, N, (float*)C, ldc, alpha, beta, scalar_mode,
                           alpha_dev, beta_dev, epi);
    } else if (c_type == VKB_T_F16) {
        hipLaunchKernelGGL(splitk_reduce_kernel<_Float16>, dim3((uint32_t)blocks), dim3(64 * RWAVES), 0, st, P,
                           stride_split, split, M, N, (_Float16*)C, ldc, alpha, beta, scalar_mode,
                           alpha_dev, beta_dev, epi);
    } else if (c_type == VKB_T_BF16) {
        hipLaunchKernelGGL(splitk_reduce_kernel<__bf16>, dim3((uint32_t)blocks), dim3(64 * RWAVES), 0, st, P,
                           stride_split, split, M, N, (__bf16*)C, ldc, alpha, beta, scalar_mode,
                           alpha_dev, beta_dev, epi);
    } else {
        return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

extern "C" uint32_t vkb_tile_bm(int tile) {
    return tile == VKB_TILE_256 ? 256u : tile == VKB_TILE_128 ? 128u : tile == VKB_TILE_32 ? 32u : 64u;
}
extern "C" uint32_t vkb_tile_bn(int tile) { return vkb_tile_bm(tile); }
extern "C" uint32_t vkb_tile_bk(int ab_type) { return ab_type == VKB_T_F32 ? 32u : 64u; }

extern "C" int vkb_launch_gemm(const vkb_gemm_args* a, int tile, void* stream) {
    if (a->ab_type == VKB_T_F32 && a->c_type == VKB_T_F32) return vkb_launch_gemm_f32_impl(a, tile, stream);
    if (a->ab_type == VKB_T_F32 && a->c_type == VKB_T_F16) return vkb_launch_gemm_f32h_impl(a, tile, stream);
    if (a->ab_type == VKB_T_F32 && a->c_type == VKB_T_BF16) return vkb_launch_gemm_f32b_impl(a, tile, stream);
    if (a->ab_type == VKB_T_F16 && a->c_type == VKB_T_F16) return vkb_launch_gemm_f16h_impl(a, tile, stream);
    if (a->ab_type == VKB_T_F16 && a->c_type == VKB_T_F32) return vkb_launch_gemm_f16s_impl(a, tile, stream);
    if (a->ab_type == VKB_T_BF16 && a->c_type == VKB_T_BF16) return vkb_launch_gemm_bf16h_impl(a, tile, stream);
    if (a->ab_type == VKB_T_BF16 && a->c_type == VKB_T_F32) return vkb_launch_gemm_bf16s_impl(a, tile, stream);
    return (int)hipErrorInvalidValue;
}
