// skinny_f16.hip — bandwidth-bound fp16 skinny GEMM / matvec for decode.
//
// Replaces the reference's matvec family (src/vkblas.c:2100-2392, 2501-2808;
// shaders matvec_splitk_tmpl.comp, matvec_splitk_m_tmpl.comp and the
// splitk_reduce_{half,m_half}.comp reduces).  The reference could only reach
// its matvec for the decode layout (hipBLAS TA=T: each output's K weights
// contiguous) through a cached transposed copy of the weight
// (VKBLAS_CACHE_TRANSPOSE, src/vkblas.c:3543-3554, 1670-1691); here that layout
// is the native one.
//
//   C[m][n] = alpha * sum_k X[m][k] * W[n][k] + beta * C[m][n],  m < M <= 16
//
// Work decomposition: a workgroup owns R tiles of 16 weight rows; its WAVES
// waves split K into contiguous slices.  Per 128-wide K step a lane streams
// 64 contiguous bytes of one weight row (four 16-byte loads) and the matching
// 64 bytes of one activation row, and feeds four v_mfma_f32_16x16x32_f16 per
// row tile (src A = 16 weight rows, src B = up to 16 activation rows; unused
// activation rows are zero).  Lane group g = lane/16 owns k in
// [128 c + 32 g, 128 c + 32 g + 32); MFMA j of the step takes the j-th 8 of
// those, the same k for both operands, so every k is used exactly once.
// The waves' 16x16 partial tiles are summed in LDS in wave order (fixed
// order: deterministic), then alpha / beta are applied once.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "vkb_launch.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct SkParams {
    const _Float16* X;
    const _Float16* W;
    void* C;
    int64_t lda, ldb, ldc;
    uint32_t M, N, K;
    float alpha, beta;
    int mode;
    const void* alpha_dev;
    const void* beta_dev;
};

__device__ __forceinline__ u32x4 ld8_checked(const _Float16* p, int nvalid) {
    if (nvalid >= 8) return *(const u32x4*)p;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i)
        if (i < nvalid) w[i >> 1] |= (uint32_t)(*(const uint16_t*)(p + i)) << (16 * (i & 1));
    return u32x4{w[0], w[1], w[2], w[3]};
}

template <typename TC, int R, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void skinny_f16_kernel(SkParams p) {
    __shared__ float red[WAVES][R][4][64];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * 16 * R;

    const int nsteps = (int)((p.K + 127) / 128);
    const int full_steps = (int)(p.K / 128);
    const int per = (nsteps + WAVES - 1) / WAVES;
    const int c_beg = wave * per;
    const int c_end = min(nsteps, c_beg + per);

    const bool xok = l16 < (int)p.M;
    const _Float16* xp = p.X + (int64_t)(xok ? l16 : 0) * p.lda + g * 32;
    const _Float16* wp[R];
    bool wok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = n0 + r * 16 + l16;
        wok[r] = row < (int)p.N;
        wp[r] = p.W + (int64_t)(wok[r] ? row : 0) * p.ldb + g * 32;
    }

    floatx4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = floatx4{0.f, 0.f, 0.f, 0.f};

    const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
    int c = c_beg;
    const int c_full_end = min(c_end, full_steps);
    // main loop: two 128-wide K steps per iteration, all loads issued first
    for (; c + 2 <= c_full_end; c += 2) {
        u32x4 xv[2][4], wv[2][R][4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t kb = (int64_t)(c + u) * 128;
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    wv[u][r][j] = wok[r] ? *(const u32x4*)(wp[r] + kb + j * 8) : zero;
#pragma unroll
            for (int j = 0; j < 4; ++j) xv[u][j] = xok ? *(const u32x4*)(xp + kb + j * 8) : zero;
        }
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < R; ++r)
                    acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        __builtin_bit_cast(half8_t, wv[u][r][j]), __builtin_bit_cast(half8_t, xv[u][j]), acc[r], 0, 0, 0);
    }
    // remaining steps, including a partial last step (zero-filled beyond K)
    for (; c < c_end; ++c) {
        const int kb = c * 128;
        u32x4 xv[4], wv[R][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int nvalid = (int)p.K - (kb + g * 32 + j * 8);
#pragma unroll
            for (int r = 0; r < R; ++r) wv[r][j] = wok[r] ? ld8_checked(wp[r] + kb + j * 8, nvalid) : zero;
            xv[j] = xok ? ld8_checked(xp + kb + j * 8, nvalid) : zero;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < R; ++r)
                acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    __builtin_bit_cast(half8_t, wv[r][j]), __builtin_bit_cast(half8_t, xv[j]), acc[r], 0, 0, 0);
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[wave][r][e][lane] = acc[r][e];
    __syncthreads();

    float alpha = p.alpha, beta = p.beta;
    if (p.mode == 1) {
        alpha = *(const float*)p.alpha_dev;
        beta = *(const float*)p.beta_dev;
    } else if (p.mode == 2) {
        alpha = (float)*(const _Float16*)p.alpha_dev;
        beta = (float)*(const _Float16*)p.beta_dev;
    }
    // output (t, o): MFMA tile r = o / 16, D row = o % 16 = 4 g + e, column t
    const int rows = 16 * R;
    for (int idx = tid; idx < (int)p.M * rows; idx += WAVES * 64) {
        const int t = idx / rows, ol = idx - t * rows;
        const int o = n0 + ol;
        if (o >= (int)p.N) continue;
        const int r = ol >> 4, dr = ol & 15;
        const int src_lane = (dr >> 2) * 16 + t, e = dr & 3;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) s += red[w][r][e][src_lane];
        TC* dst = (TC*)p.C + (int64_t)t * p.ldc + o;
        float y = alpha * s;
        if (beta != 0.0f) y += beta * (float)*dst;
        *dst = (TC)y;
    }
}

template <typename TC, int R, int WAVES>
int launch_sk(const SkParams& p, hipStream_t st) {
    const uint32_t grid = (p.N + 16 * R - 1) / (16 * R);
    hipLaunchKernelGGL((skinny_f16_kernel<TC, R, WAVES>), dim3(grid), dim3(WAVES * 64), 0, st, p);
    return (int)hipGetLastError();
}

}  // namespace

extern "C" int vkb_launch_skinny_f16(const void* X, int64_t lda, const void* W, int64_t ldb,
                                     void* C, int64_t ldc, int c_type,
                                     uint32_t M, uint32_t N, uint32_t K,
                                     float alpha, float beta, int scalar_mode,
                                     const void* alpha_dev, const void* beta_dev, void* stream) {
    if (M == 0 || M > 16 || N == 0 || K == 0) return (int)hipErrorInvalidValue;
    if ((lda & 7) || (ldb & 7) || ((uintptr_t)X & 15) || ((uintptr_t)W & 15)) return (int)hipErrorInvalidValue;
    SkParams p;
    p.X = (const _Float16*)X; p.W = (const _Float16*)W; p.C = C;
    p.lda = lda; p.ldb = ldb; p.ldc = ldc;
    p.M = M; p.N = N; p.K = K;
    p.alpha = alpha; p.beta = beta; p.mode = scalar_mode;
    p.alpha_dev = alpha_dev; p.beta_dev = beta_dev;
    hipStream_t st = (hipStream_t)stream;
    // 2 row tiles per workgroup while that still leaves >= 256 workgroups
    const bool two = (N + 31) / 32 >= 256;
    if (c_type == VKB_T_F32)
        return two ? launch_sk<float, 2, 4>(p, st) : launch_sk<float, 1, 4>(p, st);
    return two ? launch_sk<_Float16, 2, 4>(p, st) : launch_sk<_Float16, 1, 4>(p, st);
}
