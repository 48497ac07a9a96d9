// skinny.hip — bandwidth-bound skinny GEMM / matvec for decode (fp16, bf16, fp32).
//
// Replaces the reference's matvec family (src/vkblas.c:2100-2392, 2501-2808;
// shaders matvec_splitk_tmpl.comp, matvec_splitk_m_tmpl.comp and the
// splitk_reduce_{half,m_half}.comp reduces).  The reference could only reach
// its matvec for the decode layout (hipBLAS TA=T: each output's K weights
// contiguous) through a cached transposed copy of the weight
// (VKBLAS_CACHE_TRANSPOSE, src/vkblas.c:3543-3554, 1670-1691); here that layout
// is the native one.
//
//   C[m][n] = alpha * sum_k X[m][k] * W[n][k] + beta * C[m][n],  m < M <= 64
//
// Three kernels by the number of activation rows M:
//  * M == 1: gemv_kernel, v_dot2 accumulation on whole-row loads;
//  * 2 <= M <= 16: skinny_lds_kernel, one v_mfma_f32_16x16x32_{f16,bf16}
//    tile (src A = 16 weight rows, src B = up to 16 activation rows) whose
//    operands are copied to LDS as whole lines and read back as fragments;
//  * 17 <= M <= 64: decode_lds_kernel (16-bit types and fp32), weights and
//    activations copied to a shared LDS stage as whole lines (activations
//    read from L2 once per 128 weight rows), K split over the grid.
// Lane group g = lane / 16 of MFMA j takes k in [32 j + 8 g, +8) of a step:
// the same k for both operands, every k exactly once.  Partial tiles are
// summed in a fixed order (deterministic), then alpha / beta are applied once.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "epilogue.hpp"
#include "vkb_launch.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Element type T of X and W (_Float16 or __bf16): the two 16-bit products.
template <typename T>
__device__ __forceinline__ floatx4 mfma16(u32x4 a, u32x4 b, floatx4 c) {
    if constexpr (__is_same(T, __bf16))
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                      __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
}

// The MFMAs of one 16-byte fragment pair (lane group g = lane / 16 holds the
// g-th 16 bytes of a 64-byte k slice for its row): 16-bit types one
// v_mfma_f32_16x16x32 (8 k per lane), fp32 four v_mfma_f32_16x16x4_f32, the
// c-th taking element c of every lane's 4 (k = 4 g + c: each k of the slice
// exactly once, in the same order for both operands).
template <typename T>
__device__ __forceinline__ floatx4 mfma_frag(u32x4 a, u32x4 b, floatx4 c) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[e]), __uint_as_float(b[e]), c, 0, 0, 0);
        return c;
    } else {
        return mfma16<T>(a, b, c);
    }
}

// 16 bytes of T elements from p, element i zero unless i < nvalid
template <typename T>
__device__ __forceinline__ u32x4 ld16_checked(const T* p, int nvalid) {
    if (nvalid >= (int)(16 / sizeof(T))) return *(const u32x4*)p;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if constexpr (sizeof(T) == 4) {
        const uint32_t* q = (const uint32_t*)p;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < nvalid) w[i] = q[i];
    } else {
        const uint16_t* q = (const uint16_t*)p;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (i < nvalid) w[i >> 1] |= (uint32_t)q[i] << (16 * (i & 1));
    }
    return u32x4{w[0], w[1], w[2], w[3]};
}

// a + w.lo * x.lo + w.hi * x.hi (v_dot2_f32_f16 / v_dot2c_f32_bf16)
template <typename T>
__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float a) {
    if constexpr (__is_same(T, __bf16))
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, x), a,
                                               false);
    else
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w), __builtin_bit_cast(half2_t, x), a, false);
}

// decode_lds_kernel from this many activation rows on
constexpr int DEC_MIN_M = 17;

// decode_lds_kernel geometry: R 16-row weight tiles per wave (64 R rows per
// workgroup, R = 1 or 2) and the K split.  R = 2 (one workgroup per CU) when
// its grid fills at least 240 of the 256 CUs in one round; otherwise R = 1,
// whose smaller workgroups (two per CU up to 32 activation rows) spread the
// same work over more slots.  Measured: 8192x8192 n = 17-64 R = 2 27.0-32.5
// us against R = 1 36.4-45.8 us; K=4096, O=14336 (R = 2 fills 224 CUs) R = 2
// 30.3-35.5 us against R = 1 24.5-34.3 us.  The split is the largest that
// keeps the grid within one round (256 or 512 workgroups), with at least 4 K
// steps per slice: a second round costs more than its shorter slices save,
// and slices of a few steps are dominated by filling and draining the copy
// pipeline.
struct DecPlan {
    int r;
    uint32_t split;
};
__host__ __device__ inline DecPlan dec_plan(uint32_t N, uint32_t K, uint32_t es) {
    const uint32_t ks = 256 / es;   // k per step
    const uint32_t nsteps = (K + ks - 1) / ks;
    auto split_for = [&](uint32_t wg, uint32_t round) {
        uint32_t sp = round / (wg ? wg : 1);
        if (sp > nsteps / 4) sp = nsteps / 4;
        if (sp > 64) sp = 64;
        if (sp < 1) sp = 1;
        const uint32_t per = (nsteps + sp - 1) / sp;   // every slice non-empty
        return (nsteps + per - 1) / per;
    };
    const uint32_t wg2 = (N + 127) / 128;
    const uint32_t s2 = split_for(wg2, 256);
    if ((uint64_t)wg2 * s2 >= 240) return DecPlan{2, s2};
    return DecPlan{1, split_for((N + 63) / 64, 512)};
}

struct SkParams {
    const void* X;       // elements of the input type (fp32, or fp16 / bf16 bits)
    const void* W;
    void* C;
    int64_t lda, ldb, ldc;
    uint32_t M, N, K;
    float alpha, beta;
    int mode;
    const void* alpha_dev;
    const void* beta_dev;
    vkb::EpiParams epi;   // Cin (beta's matrix) and bias per output column o
};

// ------------------------------------------------------- staged skinny
// For 3 <= M <= 16 activation rows, full-line loads.  Loading the MFMA
// fragment layout directly takes 64 bytes of each of 16 weight rows per
// instruction, which measured 0.6-0.7 of HBM bandwidth; here every load is a
// buffer-to-LDS copy (buffer_load_dwordx4 ...
// lds: lane l writes 16 B at M0 + 16 l) of 4 rows x 256 contiguous bytes,
// whole 128-byte lines streamed non-temporal, and the fragments are read back
// from LDS.
// Workgroup: R 16-row weight tiles (R = 1 or 2), WAVES waves (4, or 2 for
// short K) splitting the full 128-wide K steps into contiguous slices; each wave walks its
// slice from a step rotated by workgroup (measured: without the rotation,
// workgroups that read the same column range of their rows at once lose a
// quarter of the bandwidth).  Per step a wave copies the 16 R weight rows
// (4 R instructions) and XR = 8 or 16 activation rows (XR / 4 instructions; rows
// past M repeat row M - 1, their outputs are dropped) into one of its own S
// LDS stages, S steps in flight, and waits for the oldest with
// s_waitcnt vmcnt: only the wave reads its stages, so the loop has no
// barrier.  Stage layout: rows of 256 bytes (weights, then activations),
// 16-byte unit u of row r at slot u ^ (r & 15), so the 16 rows of a fragment
// read fall on 16 distinct 16-byte bank groups.  Fragment j of a step is
// MFMA j: lane group g takes k [32 j + 8 g, +8) of both operands.
// The DMA is inline assembly (M0 operand): the compiler's own LDS DMA makes
// it wait for every copy in flight before each LDS read.  Copies read whole
// rows of full steps only, rows past N repeat the tile's last row, and the
// partial last step (K % 128) goes through plain checked loads.
template <typename T, typename TC, int XR, int S, int R, int WAVES = 4>
__global__ __launch_bounds__(64 * WAVES) void skinny_lds_kernel(SkParams p) {
    constexpr int ES = sizeof(T);                   // element bytes: 2, or 4 for fp32
    constexpr int KS = 256 / ES;                    // elements of a 256-byte K step
    constexpr int NQX = XR / 4, NQ = 4 * R + NQX;   // copies per step
    constexpr int WR = 16 * R;                      // weight rows per workgroup
    constexpr int STG = (WR + XR) * 256;            // stage bytes
    static_assert(XR == 4 || XR == 8 || XR == 16, "activation rows staged: 4, 8 or 16");
    static_assert(S >= 2 && S <= 4 && (S - 1) * NQ < 64 && WAVES * S * STG <= 160 * 1024, "stages");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[WAVES * S * STG];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * WR;
    const int rows_here = min(WR, (int)p.N - n0);

    const int nfull = (int)(p.K / KS);
    const int per = (nfull + WAVES - 1) / WAVES;
    const int c_beg = min(nfull, wave * per);
    const int n = min(nfull, c_beg + per) - c_beg;   // wave-uniform

    auto rsrc_words = [](const void* base, int64_t bytes) {
        const uint64_t a = (uint64_t)base;
        return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                     __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32) & 0xffff),
                     __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
    };
    // ranges: the operands' read domains
    const T* Wt = (const T*)p.W;
    const T* Xt = (const T*)p.X;
    const i32x4 rw = rsrc_words(Wt + (int64_t)n0 * p.ldb, ((int64_t)(rows_here - 1) * p.ldb + p.K) * ES);
    const i32x4 rx = rsrc_words(Xt, ((int64_t)(p.M - 1) * p.lda + p.K) * ES);
    int vw[4 * R], vx[NQX];
#pragma unroll
    for (int q = 0; q < 4 * R; ++q) {
        const int row = 4 * q + g;
        vw[q] = (int)((int64_t)min(row, rows_here - 1) * p.ldb * ES) + ((l16 ^ (row & 15)) << 4);
    }
#pragma unroll
    for (int q = 0; q < NQX; ++q) {
        const int t = 4 * q + g;
        vx[q] = (int)((int64_t)min(t, (int)p.M - 1) * p.lda * ES) + ((l16 ^ t) << 4);
    }
    uint8_t* my = lds + wave * S * STG;
    const int rot = n > 0 ? (int)((blockIdx.x * 7u) % (uint32_t)n) : 0;
    auto copy_step = [&](int i, int stage) {
        int q = i + rot;
        if (q >= n) q -= n;
        const int kb = __builtin_amdgcn_readfirstlane((c_beg + q) * 256);
        uint8_t* st = my + stage * STG;
#pragma unroll
        for (int c = 0; c < 4 * R; ++c) {
            const int m0 = __builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(st + c * 1024));
            asm volatile("buffer_load_dwordx4 %0, %1, %2 offen nt lds" ::"v"(vw[c]), "s"(rw), "s"(kb), "{m0}"(m0)
                         : "memory");
        }
#pragma unroll
        for (int c = 0; c < NQX; ++c) {
            const int m0 = __builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(st + WR * 256 + c * 1024));
            asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(vx[c]), "s"(rx), "s"(kb), "{m0}"(m0)
                         : "memory");
        }
    };

    floatx4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < S && i < n; ++i) copy_step(i, i);
    int stage = 0;
    for (int i = 0; i < n; ++i) {
        // step i's copies are complete once at most `later` steps' remain
        const int later = min(S - 1, n - 1 - i);
        if (later == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        else if (later == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NQ) : "memory");
        else if (later == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NQ) : "memory");
        else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * NQ) : "memory");
        const uint8_t* st = my + stage * STG;
        // MFMA columns t >= XR (never stored: XR >= M) repeat row t % XR
        const int xrow = l16 & (XR - 1);
        u32x4 wf[R][4], xf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int slot = ((4 * j + g) ^ l16) << 4;
#pragma unroll
            for (int r = 0; r < R; ++r) wf[r][j] = *(const u32x4*)(st + (16 * r + l16) * 256 + slot);
            xf[j] = *(const u32x4*)(st + WR * 256 + xrow * 256 + (((4 * j + g) ^ xrow) << 4));
        }
        // the stage is refilled only after its reads have returned
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (i + S < n) copy_step(i + S, stage);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = mfma_frag<T>(wf[r][j], xf[j], acc[r]);
        stage = stage + 1 == S ? 0 : stage + 1;
    }

    // partial last K step (zero-filled beyond K): the last wave, plain loads
    if (wave == WAVES - 1 && (p.K % KS)) {
        constexpr int FE = 16 / ES;                 // elements per 16-byte fragment unit
        const int kb = nfull * KS;
        const bool xok = l16 < (int)p.M;
        const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
        u32x4 xt[4], wt[R][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = kb + (4 * j + g) * FE;
            const int nvalid = (int)p.K - k;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = n0 + 16 * r + l16;
                wt[r][j] = row < (int)p.N ? ld16_checked<T>(Wt + (int64_t)row * p.ldb + k, nvalid) : zero;
            }
            xt[j] = xok ? ld16_checked<T>(Xt + (int64_t)l16 * p.lda + k, nvalid) : zero;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r] = mfma_frag<T>(wt[r][j], xt[j], acc[r]);
    }

    // the stages become the reduce buffer once every wave is done with them
    __syncthreads();
    float(*red)[R][4][64] = (float(*)[R][4][64])lds;
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
    // output (t, o): tile r = o / 16, D row o % 16 = 4 g + e, column t
    for (int idx = tid; idx < (int)p.M * WR; idx += 64 * WAVES) {
        const int t = idx / WR, ol = idx - t * WR;
        const int o = n0 + ol;
        if (o >= (int)p.N) continue;
        const int r = ol >> 4, dr = ol & 15;
        const int src_lane = (dr >> 2) * 16 + t, e = dr & 3;
        float s = red[0][r][e][src_lane];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) s += red[w][r][e][src_lane];
        TC* dst = (TC*)p.C + (int64_t)t * p.ldc + o;
        float y = alpha * s;
        if (beta != 0.0f) y += beta * (float)((const TC*)p.epi.cin)[(int64_t)t * p.epi.ldcin + o];
        if (p.epi.bias) y += vkb::bias_at(p.epi, o);
        *dst = (TC)y;
    }
}

// ---------------------------------------------------------------- GEMV
// For one activation row (token-by-token decode) the MFMA tile is mostly
// idle and its fragment layout splits every load over 16 rows (half lines).
// Here a wave reads 1 KB of ONE weight row per instruction (8 whole 128-byte
// lines, loaded non-temporal: the weights stream through once, and whole-line
// requests let nt skip the cache without re-fetching the other half of a
// line): lane l takes k in [c*512 + 8 l, +8) of chunk c and multiplies it
// with the same k of each activation row (v_dot2_f32_f16 / v_dot2c_f32_bf16,
// fp32 accumulate).
// Workgroup: 4 waves, RB weight rows; wave w takes chunks w, w+4, ... of K,
// loading the next chunk's RB rows while it computes the current one.
// Partials (MM x RB per lane) are summed across the 64 lanes by a butterfly
// reduce-scatter, then across the 4 waves in wave order: deterministic.
template <typename T, typename TC, int MM, int RB>
__global__ __launch_bounds__(256) void gemv_kernel(SkParams p) {
    constexpr int P = MM * RB;                    // partials per lane (power of 2, <= 64)
    constexpr int LP = P == 2 ? 1 : P == 4 ? 2 : P == 8 ? 3 : P == 16 ? 4 : P == 32 ? 5 : 6;
    static_assert((1 << LP) == P, "MM * RB must be a power of 2 in [2, 64]");
    __shared__ float red[4][P];
    const uint16_t* pX = (const uint16_t*)p.X;
    const uint16_t* pW = (const uint16_t*)p.W;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * RB;
    const int rows_here = min(RB, (int)p.N - n0);
    // The buffer ranges are exactly the operands' read domains ((rows - 1) ld
    // + K elements): rows past N, activation rows past M and k past K in the
    // last row read as zero and never touch memory beyond the allocation.
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(pW + (int64_t)n0 * p.ldb), (short)0, (int)(((int64_t)(rows_here - 1) * p.ldb + p.K) * 2),
        0x00020000);
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        (void*)pX, (short)0, (int)(((int64_t)(p.M - 1) * p.lda + p.K) * 2), 0x00020000);
    const int nch = (int)((p.K + 511) / 512);

    float acc[MM][RB];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[m][r] = 0.0f;

    u32x4 wc[RB], xc[MM];
    auto load = [&](int c, u32x4* w, u32x4* x) {
        const int kb = (c * 512 + lane * 8) * 2;   // byte offset within a row
#pragma unroll
        for (int m = 0; m < MM; ++m) x[m] = __builtin_amdgcn_raw_buffer_load_b128(rx, m * (int)p.lda * 2 + kb, 0, 0);
#pragma unroll
        for (int r = 0; r < RB; ++r)   // streamed once: non-temporal (nt)
            w[r] = __builtin_amdgcn_raw_buffer_load_b128(rw, r * (int)p.ldb * 2 + kb, 0, 2);
    };
    auto compute = [&](int c, const u32x4* w, const u32x4* x) {
        // lanes past K (last chunk) contribute nothing; the padding past K
        // may hold anything (NaN), so both operands are zeroed.  The lane
        // whose 8 elements straddle K (K % 8 != 0) reloads them element by
        // element, zero past K.
        const int k = c * 512 + lane * 8;
        const int nvalid = (int)p.K - k;
        const bool valid = nvalid > 0;
        const u32x4 z = u32x4{0u, 0u, 0u, 0u};
        u32x4 ws[RB], xs[MM];
#pragma unroll
        for (int r = 0; r < RB; ++r) ws[r] = w[r];
#pragma unroll
        for (int m = 0; m < MM; ++m) xs[m] = x[m];
        if (valid && nvalid < 8) {
#pragma unroll
            for (int r = 0; r < RB; ++r)
                ws[r] = r < rows_here ? ld16_checked(pW + (int64_t)(n0 + r) * p.ldb + k, nvalid) : z;
#pragma unroll
            for (int m = 0; m < MM; ++m) xs[m] = ld16_checked(pX + (int64_t)m * p.lda + k, nvalid);
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const u32x4 wr = valid ? ws[r] : z;
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                const u32x4 xm = valid ? xs[m] : z;
                float a = acc[m][r];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // element copied out first: a bit cast of a vector
                    // subscript compiled to element 0 for every e
                    const uint32_t we = wr[e], xe = xm[e];
                    a = dot2<T>(we, xe, a);
                }
                acc[m][r] = a;
            }
        }
    };
    int c = wave;
    if (c < nch) load(c, wc, xc);
    for (; c < nch; c += 4) {
        u32x4 wn[RB], xn[MM];
        const bool more = c + 4 < nch;
        if (more) load(c + 4, wn, xn);
        compute(c, wc, xc);
        if (more) {
#pragma unroll
            for (int r = 0; r < RB; ++r) wc[r] = wn[r];
#pragma unroll
            for (int m = 0; m < MM; ++m) xc[m] = xn[m];
        }
    }

    // butterfly reduce-scatter over lane bits 0 .. LP-1, then a plain
    // butterfly over the rest: lane l ends with the 64-lane total of
    // partial j(l) = sum_t bit_t(l) * (P >> (t + 1)).
    float v[P];
#pragma unroll
    for (int m = 0; m < MM; ++m)
#pragma unroll
        for (int r = 0; r < RB; ++r) v[m * RB + r] = acc[m][r];
#pragma unroll
    for (int t = 0; t < LP; ++t) {
        const int H = P >> (t + 1);
        const bool upper = (lane >> t) & 1;
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const float send = upper ? v[i] : v[i + H];
            const float keep = upper ? v[i + H] : v[i];
            v[i] = keep + __shfl_xor(send, 1 << t);
        }
    }
#pragma unroll
    for (int t = LP; t < 6; ++t) v[0] += __shfl_xor(v[0], 1 << t);
    if (lane < P) {
        int j = 0;
#pragma unroll
        for (int t = 0; t < LP; ++t) j += ((lane >> t) & 1) * (P >> (t + 1));
        red[wave][j] = v[0];
    }
    __syncthreads();

    if (tid < P) {
        const int m = tid / RB, r = tid % RB;
        if (m < (int)p.M && n0 + r < (int)p.N) {
            float alpha = p.alpha, beta = p.beta;
            if (p.mode == 1) {
                alpha = *(const float*)p.alpha_dev;
                beta = *(const float*)p.beta_dev;
            } else if (p.mode == 2) {
                alpha = (float)*(const _Float16*)p.alpha_dev;
                beta = (float)*(const _Float16*)p.beta_dev;
            }
            const float s = ((red[0][tid] + red[1][tid]) + red[2][tid]) + red[3][tid];
            TC* dst = (TC*)p.C + (int64_t)m * p.ldc + n0 + r;
            float y = alpha * s;
            if (beta != 0.0f) y += beta * (float)((const TC*)p.epi.cin)[(int64_t)m * p.epi.ldcin + n0 + r];
            if (p.epi.bias) y += vkb::bias_at(p.epi, n0 + r);
            *dst = (TC)y;
        }
    }
}

// ------------------------------------------------------- staged decode
// For 17 <= M <= 64 activation rows, fp16 / bf16 or fp32.  The workgroup owns 64 R weight rows
// (wave w computes rows 16 R w .. 16 R w + 16 R - 1: R 16-row tiles, R = 1
// or 2, see dec_plan) against all 16 MT activation rows (MT = ceil(M / 16)
// tiles), and the grid splits K
// over blockIdx.y: with nsplit > 1 each workgroup writes raw fp32 partials
// (part + split * M * N, row pitch N) that splitk_reduce sums in split order.
// Per K step (256 bytes of each row: 128 k of a 16-bit type, one
// v_mfma_f32_16x16x32 per fragment; 64 k of fp32, four v_mfma_f32_16x16x4f32
// per fragment, see mfma_frag) the workgroup copies its weight rows and the
// activation rows into one shared LDS stage as whole 256-byte row pieces
// (buffer_load_dwordx4 ... lds, 4 rows per instruction; wave w copies its own
// weight rows and a quarter of the activation rows), S stages, S - 1 steps in
// flight; each wave waits for its own copies of the oldest step with
// s_waitcnt vmcnt, then a barrier makes the stage complete.  The activations
// are read from L2 once per 64 R weight rows.  Stage layout: rows of 256
// bytes (weights, then activations), unit u of row r at slot u ^ (r & 15):
// fragment reads of 16 consecutive rows are conflict-free.  Rows past N / M
// repeat the last row (outputs dropped); the partial last K step goes through
// plain checked loads.
template <typename T, typename TC, int R, int MT, int S, bool PARTIAL>
__global__ __launch_bounds__(256) void decode_lds_kernel(SkParams p, float* part, int nsplit) {
    constexpr int WROWS = 64 * R;             // weight rows per workgroup
    constexpr int NQ = 4 * R + MT;            // copies per wave and step
    constexpr int STG = (WROWS + 16 * MT) * 256;
    static_assert(S >= 2 && S <= 4 && S * STG <= 160 * 1024 && (S - 2) * NQ < 64, "stages");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S * STG];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, g = lane >> 4;
    const int N = (int)p.N, M = (int)p.M, K = (int)p.K;
    constexpr int ES = (int)sizeof(T), KS = 256 / ES;        // element bytes, k per step
    const T* pX = (const T*)p.X;
    const T* pW = (const T*)p.W;
    const int wrow0 = blockIdx.x * WROWS + wave * 16 * R;     // this wave's first weight row
    const int nsteps = (K + KS - 1) / KS, full_steps = K / KS;
    const int per = (nsteps + nsplit - 1) / nsplit;
    const int s_beg = (int)blockIdx.y * per;
    const int s_end = min(nsteps, s_beg + per);
    const int n = max(0, min(s_end, full_steps) - s_beg);      // full steps, copied
    const bool tail = full_steps < nsteps && s_beg <= full_steps && full_steps < s_end;

    auto rsrc_words = [](const void* base, int64_t bytes) {
        const uint64_t a = (uint64_t)base;
        return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                     __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32) & 0xffff),
                     __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
    };
    // weight buffer on the wave's first row (clamped to the last row), range
    // the read domain of the rows it copies
    const int wbase = min(wrow0, N - 1);
    const int wlast = min(wrow0 + 16 * R - 1, N - 1);
    const i32x4 rw = rsrc_words(pW + (int64_t)wbase * p.ldb, ((int64_t)(wlast - wbase) * p.ldb + K) * ES);
    const i32x4 rx = rsrc_words(pX, ((int64_t)(M - 1) * p.lda + K) * ES);
    int vw[4 * R], vx[MT];
#pragma unroll
    for (int q = 0; q < 4 * R; ++q) {
        const int rr = 4 * q + g;                               // row within the wave's 16 R
        vw[q] = (int)((int64_t)(min(wrow0 + rr, N - 1) - wbase) * p.ldb * ES) + ((l16 ^ (rr & 15)) << 4);
    }
#pragma unroll
    for (int q = 0; q < MT; ++q) {
        const int xr = wave * 4 * MT + 4 * q + g;               // activation row
        vx[q] = (int)((int64_t)min(xr, M - 1) * p.lda * ES) + ((l16 ^ (xr & 15)) << 4);
    }
    // the workgroups of a K slice walk it from rotated starts, so they do
    // not all read the same column range of their rows at once
    const int rot = n > 0 ? (int)((blockIdx.x * 7u) % (uint32_t)n) : 0;
    auto step_kb = [&](int i) {
        const int q0 = i + rot;
        return __builtin_amdgcn_readfirstlane((s_beg + (q0 >= n ? q0 - n : q0)) * 256);
    };
    // copy d of a step (d < 4 R: four weight rows, else four activation rows)
    auto copy_one = [&](int d, int kb, uint8_t* st) {
        if (d < 4 * R) {
            const int m0 = __builtin_amdgcn_readfirstlane(
                (int)(uint32_t)(uintptr_t)(st + (wave * 16 * R + 4 * d) * 256));
            asm volatile("buffer_load_dwordx4 %0, %1, %2 offen nt lds" ::"v"(vw[d]), "s"(rw), "s"(kb), "{m0}"(m0)
                         : "memory");
        } else {
            const int q = d - 4 * R;
            const int m0 = __builtin_amdgcn_readfirstlane(
                (int)(uint32_t)(uintptr_t)(st + (WROWS + wave * 4 * MT + 4 * q) * 256));
            asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(vx[q]), "s"(rx), "s"(kb), "{m0}"(m0)
                         : "memory");
        }
    };
    auto copy_step = [&](int i, int stage) {
        const int kb = step_kb(i);
        uint8_t* st = lds + stage * STG;
#pragma unroll
        for (int d = 0; d < NQ; ++d) copy_one(d, kb, st);
    };

    floatx4 acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[r][t] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (int i = 0; i < S - 1 && i < n; ++i) copy_step(i, i);
    int stage = 0;
    for (int i = 0; i < n; ++i) {
        // this wave's copies of step i are complete once at most `later`
        // steps' remain; the barrier then makes the whole stage complete and
        // ends every wave's reads of the stage refilled next
        const int later = min(S - 2, n - 1 - i);
        if (later == 0) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else if (later == 1) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(NQ) : "memory");
        else asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(2 * NQ) : "memory");
        // 16-bit: the copies of step i + S - 1 go out in one burst here.
        // fp32 (MFMA-bound from 33 rows): they go out among the first half of
        // this step's MFMAs, each product fenced by a sched_barrier: in one
        // burst they back up in the texture address unit and hold the wave's
        // MFMA issue.  Measured (8192^2, weight N x K, three weights rotated,
        // one box, two runs): fp32 32 / 64 rows 52.5-53.0 / 86.7-86.9 ->
        // 50.6-51.7 / 78.0-78.8 us (over all the MFMAs: 50.1-50.5 / 80.0-
        // 80.4); fp16 24-64 rows within 0.5 % either way.
        const bool cp = i + S - 1 < n;
        const int cstage = stage == 0 ? S - 1 : stage - 1;
        if constexpr (sizeof(T) != 4) {
            if (cp) copy_step(i + S - 1, cstage);
        }
        const uint8_t* st = lds + stage * STG;
        u32x4 wf[R][4], xf[MT][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int slot = ((4 * j + g) ^ l16) << 4;
#pragma unroll
            for (int r = 0; r < R; ++r) wf[r][j] = *(const u32x4*)(st + (wave * 16 * R + 16 * r + l16) * 256 + slot);
#pragma unroll
            for (int t = 0; t < MT; ++t) xf[t][j] = *(const u32x4*)(st + (WROWS + 16 * t + l16) * 256 + slot);
        }
        if constexpr (sizeof(T) != 4) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int t = 0; t < MT; ++t) acc[r][t] = mfma_frag<T>(wf[r][j], xf[t][j], acc[r][t]);
        } else {
            const int kb = cp ? step_kb(i + S - 1) : 0;
            uint8_t* stc = lds + cstage * STG;
            constexpr int NP = 4 * R * MT;   // fragment products per step
            int k = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int t = 0; t < MT; ++t) {
                        acc[r][t] = mfma_frag<T>(wf[r][j], xf[t][j], acc[r][t]);
                        if (cp) {
                            // copy d goes with product floor(d NP / (2 NQ))
#pragma unroll
                            for (int d = 0; d < NQ; ++d)
                                if (d * NP >= k * 2 * NQ && d * NP < (k + 1) * 2 * NQ) copy_one(d, kb, stc);
                        }
                        ++k;
                        __builtin_amdgcn_sched_barrier(0);
                    }
        }
        stage = stage + 1 == S ? 0 : stage + 1;
    }
    if (tail) {   // partial last K step, zero-filled beyond K
        const int kb = full_steps * KS;
        const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
        u32x4 wt[R][4], xt[MT][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = kb + (KS / 4) * j + (16 / ES) * g;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = wrow0 + 16 * r + l16;
                wt[r][j] = row < N ? ld16_checked(pW + (int64_t)row * p.ldb + k, K - k) : zero;
            }
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int xr = 16 * t + l16;
                xt[t][j] = xr < M ? ld16_checked(pX + (int64_t)xr * p.lda + k, K - k) : zero;
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[r][t] = mfma_frag<T>(wt[r][j], xt[t][j], acc[r][t]);
    }

    // D row 4 g + e = weight row, column l16 = activation row: each lane
    // holds four consecutive outputs of one activation row
    float alpha = p.alpha, beta = p.beta;
    if constexpr (!PARTIAL) {
        if (p.mode == 1) {
            alpha = *(const float*)p.alpha_dev;
            beta = *(const float*)p.beta_dev;
        } else if (p.mode == 2) {
            alpha = (float)*(const _Float16*)p.alpha_dev;
            beta = (float)*(const _Float16*)p.beta_dev;
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int row = 16 * t + l16;             // activation row (output row)
            const int o = wrow0 + 16 * r + 4 * g;     // first of four weight rows (output columns)
            if (row >= M) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (o + e >= N) continue;
                if constexpr (PARTIAL) {
                    part[(int64_t)blockIdx.y * M * N + (int64_t)row * N + o + e] = acc[r][t][e];
                } else {
                    TC* dst = (TC*)p.C + (int64_t)row * p.ldc + o + e;
                    float y = alpha * acc[r][t][e];
                    if (beta != 0.0f) y += beta * (float)((const TC*)p.epi.cin)[(int64_t)row * p.epi.ldcin + o + e];
                    if (p.epi.bias) y += vkb::bias_at(p.epi, o + e);
                    *dst = (TC)y;
                }
            }
        }
}

// ------------------------------------------------ fp32, W stored K x N
// C[m][n] = alpha * sum_k X[m][k] * W[k][n] + ...,  M <= 64, each W row
// N-contiguous: the reference's TB = 0 matvec (matvec_f32_tmpl.comp:27-58,
// four contiguous columns per thread), here on the matrix cores.  One
// v_mfma_f32_16x16x4_f32 takes 4 k of 16 activation rows (A operand: lane
// (l16, g) holds X[l16][k]) against the same 4 k of 16 columns (B operand:
// lane (l16, g) holds W[k][column of lane l16]).  A lane loads 16 bytes of a
// W row, columns nl .. nl + 3 with nl = n0 + 4 l16, so each load instruction
// reads 4 rows x 256 contiguous bytes (whole lines, non-temporal: the weights
// stream through once), and component c of the loads feeds tile c, whose 16
// columns are nl + c over the 16 lanes: four accumulator tiles interleaved
// over the wave's 64 columns.  A 16-row chunk is four MFMAs e per tile, MFMA
// e taking k = k0 + 4 g + e: lane group g loads W rows k0 + 4 g .. + 3 and
// X[l16][k0 + 4 g .. + 3] (one 16-byte load).  Tile c's D[i][j] sits in lane
// (j, i / 4), component i % 4, so lane (l16, g) owns C[4 g + r][nl .. nl + 3]:
// one 16-byte store per activation row.  MT activation tiles (rows 16 t ..
// 16 t + 15, M up to 16 MT) share each W fragment: acc[t][c].
// Workgroup: WV waves, WV / KW column groups of 64 side by side, KW waves
// along K splitting the workgroup's slice into contiguous parts whose sums
// are added in LDS in wave order.  Each wave loads the next chunk while it
// multiplies the current one.  grid.y splits K into slices of `per` chunks
// (PARTIAL: fp32 partials for the fixed-order reduce); the plan keeps the
// grid to one round of at most 256 workgroups, one per CU (measured on
// 8192x8192, 4096x14336 and 14336x4096: 0.74-0.82 of HBM; 384-512
// workgroups, two per CU, 0.58-0.71).  17-64 rows: four waves along K, one
// column group (the LDS sums and accumulators grow with MT); against the
// tile paths (same box, 17 / 32 / 64 rows) 14336 x 4096 56 / 58 / 85 us
// against 242 / 244 / 108, 8192^2 58 / 60 / 88 against 157 / 167 / 95.
// Requires N % 4 == 0 (lanes past N load the last 4 columns and store
// nothing), ldb % 4 == 0, lda % 4 == 0 (or M == 1) and 16-byte aligned X, W.
// Activation rows past M load row M - 1 (their outputs are dropped); k past
// K in the last chunk is zero in both operands.
constexpr int SKN_WV = 8, SKN_KW = 4;
constexpr int SKN_COLS = 64 * SKN_WV / SKN_KW;   // columns per workgroup, M <= 16
constexpr int SKN_COLS_MT = 64;                  // 17 <= M <= 64: four waves along K

template <typename TC, int WV, int KW, int MT, bool PARTIAL>
__global__ __launch_bounds__(64 * WV) void skinny_n_kernel(SkParams p, float* part, int per) {
    constexpr int CG = WV / KW;                  // column groups of 64 per workgroup
    __shared__ floatx4 red[KW > 1 ? (KW - 1) * CG * 4 * MT * 64 : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cg = wave % CG, kw = wave / CG;
    const int l16 = lane & 15, g = lane >> 4;
    const int N = (int)p.N, M = (int)p.M, K = (int)p.K;
    const int nl = blockIdx.x * (64 * CG) + cg * 64 + 4 * l16;   // this lane's columns
    const float* W = (const float*)p.W + min(nl, N - 4);
    const float* X[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) X[t] = (const float*)p.X + (int64_t)min(16 * t + l16, M - 1) * p.lda;
    const int64_t ldb = p.ldb;
    const int chunks = (K + 15) / 16;
    const int s_beg = (int)blockIdx.y * per;                      // the workgroup's slice
    const int s_end = min(chunks, s_beg + per);
    const int sub = (per + KW - 1) / KW;                          // this wave's part of it
    const int c_beg = min(s_end, s_beg + kw * sub);
    const int c_end = min(s_end, c_beg + sub);
    const int f_end = max(c_beg, min(c_end, K / 16));             // chunks with 16 valid k

    floatx4 acc[MT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[t][c] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto load = [&](int ch, floatx4 (&w)[4], floatx4 (&x)[MT]) {
        const int64_t k = (int64_t)ch * 16 + 4 * g;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = __builtin_nontemporal_load((const floatx4*)(W + (k + e) * ldb));
#pragma unroll
        for (int t = 0; t < MT; ++t) x[t] = *(const floatx4*)(X[t] + k);
    };
    auto mma = [&](const floatx4 (&w)[4], const floatx4 (&x)[MT]) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[t][e], w[e][c], acc[t][c], 0, 0, 0);
    };
    // full chunks, the next chunk's loads in flight.  (Walking them from a
    // rotated chunk, as skinny_nh_kernel does, measured 1-7 % slower here at
    // 4096 x 14336, 14336 x 4096 and 4096^2, 2-3 % faster at 8192^2 n <= 8.)
    const int nf = f_end - c_beg;
    int ch = c_beg;
    if constexpr (MT == 1) {
        floatx4 wa[4], xa[MT], wb[4], xb[MT];
        int i = 0;
        if (nf > 0) load(ch, wa, xa);
        for (; i + 1 < nf; i += 2) {
            load(ch + 1, wb, xb);
            mma(wa, xa);
            if (i + 2 < nf) load(ch + 2, wa, xa);
            mma(wb, xb);
            ch += 2;
        }
        if (i < nf) {
            mma(wa, xa);
            ++ch;
        }
    } else {
        // 17-64 rows: three chunks' loads in flight (buffer u of NB holds
        // chunk i + u).  Measured against one chunk ahead (same box, two
        // runs, 32 / 64 rows): 8192^2 60.3-60.5 / 87.8-87.9 -> 56.8-56.9 /
        // 83.5 us, K x N = 4096 x 14336 57.5-57.6 / 85.2 -> 54.9-55.0 /
        // 79.5-79.7, 14336 x 4096 54.5 / 78.3-78.7 -> 52.0-52.2 / 74.5-74.6;
        // up to 16 rows it measured -3 to +4 % and keeps one chunk ahead.
        constexpr int NB = 4;
        floatx4 wv[NB][4], xv[NB][MT];
#pragma unroll
        for (int j = 0; j < NB - 1; ++j)
            if (j < nf) load(c_beg + j, wv[j], xv[j]);
        for (int i = 0; i < nf; i += NB) {
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                if (i + u < nf) {
                    if (i + u + NB - 1 < nf) load(c_beg + i + u + NB - 1, wv[(u + NB - 1) % NB], xv[(u + NB - 1) % NB]);
                    mma(wv[u], xv[u]);
                }
            }
        }
        ch = f_end;
    }
    // the partial last chunk, k past K zero
    for (; ch < c_end; ++ch) {
        const int k = ch * 16 + 4 * g;
        floatx4 w[4], x[MT];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const bool ok = k + e < K;
            w[e] = ok ? *(const floatx4*)(W + (int64_t)(k + e) * ldb) : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < MT; ++t) x[t][e] = ok ? X[t][k + e] : 0.f;
        }
        mma(w, x);
    }
    // the KW parts of the slice, summed in wave order
    if constexpr (KW > 1) {
        if (kw > 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int c = 0; c < 4; ++c) red[((((kw - 1) * CG + cg) * MT + t) * 4 + c) * 64 + lane] = acc[t][c];
        }
        __syncthreads();
        if (kw > 0) return;
#pragma unroll
        for (int j = 1; j < KW; ++j)
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[t][c] += red[((((j - 1) * CG + cg) * MT + t) * 4 + c) * 64 + lane];
    }

    if (nl >= N) return;
    if constexpr (PARTIAL) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 16 * t + 4 * g + r;
                if (m < M)
                    *(floatx4*)(part + ((int64_t)blockIdx.y * M + m) * N + nl) =
                        floatx4{acc[t][0][r], acc[t][1][r], acc[t][2][r], acc[t][3][r]};
            }
    } else {
        float alpha = p.alpha, beta = p.beta;
        if (p.mode == 1) {
            alpha = *(const float*)p.alpha_dev;
            beta = *(const float*)p.beta_dev;
        } else if (p.mode == 2) {
            alpha = (float)*(const _Float16*)p.alpha_dev;
            beta = (float)*(const _Float16*)p.beta_dev;
        }
        float b4[4] = {0.f, 0.f, 0.f, 0.f};
        vkb::add_bias4(p.epi, nl, 4, b4);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 16 * t + 4 * g + r;
                if (m >= M) continue;
                TC* dst = (TC*)p.C + (int64_t)m * p.ldc + nl;
                const TC* src = (const TC*)p.epi.cin + (int64_t)m * p.epi.ldcin + nl;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float y = alpha * acc[t][c][r];
                    if (beta != 0.0f) y += beta * (float)src[c];
                    if (p.epi.bias) y += b4[c];
                    dst[c] = (TC)y;
                }
            }
    }
}

// 16-bit form of the N-contiguous decode (weight K x N, engine op_b = N:
// PyTorch's x @ w with w stored [K][N]).  One v_mfma_f32_16x16x32 takes 8 k
// of 16 activation rows (A: lane (l16, g) holds X[l16][k0 + 8 g .. + 7], one
// 16-byte load) against the same 8 k of 16 columns (B: lane (l16, g) holds
// W[k0 + 8 g .. + 7][column of lane l16]).  A lane loads 16 bytes (columns
// nl .. nl + 7, nl = n0 + 8 l16) of each of its 8 k rows, so a load
// instruction reads 4 rows x 256 contiguous bytes (non-temporal), and
// v_perm_b32 gathers element c of the 8 rows into the B fragment of tile c,
// whose 16 columns are nl + c over the lanes: eight accumulator tiles
// interleaved over the wave's 128 columns.  Tile c's D[i][j] sits in lane
// (j, i / 4), component i % 4, so lane (l16, g) owns C[4 g + r][nl .. nl + 7]:
// one 16-byte (16-bit C) or two (fp32 C) stores per activation row.
// MT activation tiles of 16 rows (M up to 16 MT) share each B fragment.
// Workgroup, K split and partials as skinny_n_kernel, with 32-row chunks.
// Requires N % 8 == 0 (lanes past N load the last 8 columns and store
// nothing), ldb % 8 == 0, lda % 8 == 0 (or M == 1) and 16-byte aligned X, W.
// Geometries: M <= 16 eight waves (two column groups, four along K); 17 <= M
// <= 64 four waves (one column group of 128, four along K), whose 4 MT x 8
// accumulator tiles need the register file of one wave per SIMD.
constexpr int SKH_WV = 8, SKH_KW = 4;
constexpr int SKH_COLS = 128 * SKH_WV / SKH_KW;   // columns per workgroup, M <= 16
constexpr int SKH_COLS_MT = 128;                  // columns per workgroup, M > 16

template <typename T, typename TC, int WV, int KW, int MT, bool PARTIAL>
__global__ __launch_bounds__(64 * WV) void skinny_nh_kernel(SkParams p, float* part, int per) {
    constexpr int CG = WV / KW;                  // column groups of 128 per workgroup
    __shared__ floatx4 red[KW > 1 ? (KW - 1) * CG * MT * 8 * 64 : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int cg = wave % CG, kw = wave / CG;
    const int l16 = lane & 15, g = lane >> 4;
    const int N = (int)p.N, M = (int)p.M, K = (int)p.K;
    const int nl = blockIdx.x * (128 * CG) + cg * 128 + 8 * l16;  // this lane's columns
    const T* W = (const T*)p.W + min(nl, N - 8);
    const T* X[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) X[t] = (const T*)p.X + (int64_t)min(16 * t + l16, M - 1) * p.lda;
    const int64_t ldb = p.ldb;
    const int chunks = (K + 31) / 32;
    const int s_beg = (int)blockIdx.y * per;                      // the workgroup's slice
    const int s_end = min(chunks, s_beg + per);
    const int sub = (per + KW - 1) / KW;                          // this wave's part of it
    const int c_beg = min(s_end, s_beg + kw * sub);
    const int c_end = min(s_end, c_beg + sub);
    const int f_end = max(c_beg, min(c_end, K / 32));             // chunks with 32 valid k

    floatx4 acc[MT][8];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[t][c] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto load = [&](int ch, u32x4 (&w)[8], u32x4 (&x)[MT]) {
        const int64_t k = (int64_t)ch * 32 + 8 * g;
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = __builtin_nontemporal_load((const u32x4*)(W + (k + e) * ldb));
#pragma unroll
        for (int t = 0; t < MT; ++t) x[t] = *(const u32x4*)(X[t] + k);
    };
    // tile c: element c of the 8 rows, rows 2 d and 2 d + 1 in dword d
    auto mma = [&](const u32x4 (&w)[8], const u32x4 (&x)[MT]) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
            u32x4 b;
#pragma unroll
            for (int d = 0; d < 4; ++d) b[d] = __builtin_amdgcn_perm(w[2 * d + 1][c >> 1], w[2 * d][c >> 1], sel);
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[t][c] = mfma16<T>(x[t], b, acc[t][c]);
        }
    };
    // full chunks, the next chunk's loads in flight.  Each workgroup walks
    // them from a chunk rotated by its position in the grid: the workgroups
    // of one K slice (every column block) then read different weight rows at
    // a time instead of the same ones.  Streaming probe (8192^2 fp16, three
    // weights rotated): 6.0 -> 6.5 TB/s; this kernel, same box, A/B: 8192^2
    // n = 1 / 8 / 16 27.2 / 27.7 / 28.1 -> 24.7 / 25.1 / 25.5 us, 4096^2
    // 11.5-12.6 -> 10.4-11.6, 14336 x 4096 (K x N) -1 %, 4096 x 14336 +1-2 %.
    const int nf = f_end - c_beg;
    const int rot = nf > 0 ? (int)((blockIdx.x * 7u + blockIdx.y * 3u) % (uint32_t)nf) : 0;
    auto cidx = [&](int i) { return c_beg + (i + rot < nf ? i + rot : i + rot - nf); };
    {
        u32x4 wa[8], xa[MT], wb[8], xb[MT];
        int i = 0;
        if (nf > 0) load(cidx(0), wa, xa);
        for (; i + 1 < nf; i += 2) {
            load(cidx(i + 1), wb, xb);
            mma(wa, xa);
            if (i + 2 < nf) load(cidx(i + 2), wa, xa);
            mma(wb, xb);
        }
        if (i < nf) mma(wa, xa);
    }
    int ch = f_end;
    // the partial last chunk, k past K zero in both operands
    for (; ch < c_end; ++ch) {
        const int k = ch * 32 + 8 * g;
        u32x4 w[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            w[e] = k + e < K ? *(const u32x4*)(W + (int64_t)(k + e) * ldb) : u32x4{0u, 0u, 0u, 0u};
        u32x4 x[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) x[t] = ld16_checked<T>(X[t] + k, K - k);
        mma(w, x);
    }
    // the KW parts of the slice, summed in wave order
    if constexpr (KW > 1) {
        if (kw > 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int c = 0; c < 8; ++c) red[((((kw - 1) * CG + cg) * MT + t) * 8 + c) * 64 + lane] = acc[t][c];
        }
        __syncthreads();
        if (kw > 0) return;
#pragma unroll
        for (int j = 1; j < KW; ++j)
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int c = 0; c < 8; ++c) acc[t][c] += red[((((j - 1) * CG + cg) * MT + t) * 8 + c) * 64 + lane];
    }

    if (nl >= N) return;
    if constexpr (PARTIAL) {
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 16 * t + 4 * g + r;
                if (m < M) {
                    float* dst = part + ((int64_t)blockIdx.y * M + m) * N + nl;
                    *(floatx4*)dst = floatx4{acc[t][0][r], acc[t][1][r], acc[t][2][r], acc[t][3][r]};
                    *(floatx4*)(dst + 4) = floatx4{acc[t][4][r], acc[t][5][r], acc[t][6][r], acc[t][7][r]};
                }
            }
    } else {
        float alpha = p.alpha, beta = p.beta;
        if (p.mode == 1) {
            alpha = *(const float*)p.alpha_dev;
            beta = *(const float*)p.beta_dev;
        } else if (p.mode == 2) {
            alpha = (float)*(const _Float16*)p.alpha_dev;
            beta = (float)*(const _Float16*)p.beta_dev;
        }
        float b8[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) b8[c] = p.epi.bias ? vkb::bias_at(p.epi, nl + c) : 0.f;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = 16 * t + 4 * g + r;
                if (m >= M) continue;
                TC* dst = (TC*)p.C + (int64_t)m * p.ldc + nl;
                const TC* src = (const TC*)p.epi.cin + (int64_t)m * p.epi.ldcin + nl;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    float y = alpha * acc[t][c][r];
                    if (beta != 0.0f) y += beta * (float)src[c];
                    y += b8[c];
                    dst[c] = (TC)y;
                }
            }
    }
}

template <typename T, typename TC, int MM, int RB>
int launch_gemv(const SkParams& p, hipStream_t st) {
    const uint32_t grid = (p.N + RB - 1) / RB;
    hipLaunchKernelGGL((gemv_kernel<T, TC, MM, RB>), dim3(grid), dim3(256), 0, st, p);
    return (int)hipGetLastError();
}

// Staged skinny geometry: XR activation rows staged per step (4 for fp32 up
// to 4 rows, else 8 or 16, covering M); R 16-row weight tiles and WAVES waves
// per workgroup; S LDS stages per wave.
//  * 9-16 rows, and a grid of 32-row workgroups that fills the chip (at least
//    256): R = 2 (two tiles share every activation copy, which from 9 rows
//    weigh as much as the weight copies), two waves (each a K half), three
//    stages.  Measured (fp16, us) against R = 2 with four waves and two
//    stages: K=4096, O=14336 n = 12 / 16 21.1 / 21.9 -> 19.5 / 19.9;
//    K=8192, O=8192 n = 16 22.3 -> 21.9; K=2048, O=16384 14.1 -> 13.0;
//    K=4096, O=11008 20.5 -> 18.5; K=8192, O=28672 80.1 -> 77.6; fp32
//    K=4096, O=14336 42.0 -> 39.1.
//  * up to 8 rows of 16-bit types with 24-40 K steps, when 32-row workgroups
//    fill the chip no less evenly than 16-row ones (the busiest CU gets no
//    more rows): the same R = 2, two-wave, three-stage form.  K=4096,
//    O=14336 n = 3-8 20.6-21.1 -> 18.7-19.1 us; K=4096, O=8192 12.0-12.5 ->
//    11.8-12.3.  Not where R = 2 spreads worse (K=4096, O=11008: 16.5 ->
//    18.8), nor with 16 K steps (K=2048, O=16384: 11.6 -> 12.5) or with 64
//    (K=8192, O=8192: 21.0 -> 22.0), nor for fp32 (K=2048, O=16384 n = 8:
//    21.2 -> 23.0).
//  * otherwise one tile, two stages; up to 8 rows two waves per workgroup
//    (each a K half) when four would leave each wave fewer than 16 K steps
//    and the grid has at least 512 workgroups (measured, n = 3-8: K=4096,
//    O=14336 21.6 -> 19.5 us, K=4096, O=8192 12.3-12.8 -> 11.7 us), else
//    four waves.
struct SklPlan {
    int xr, r, waves, stages;
};
inline SklPlan skl_plan(uint32_t es, uint32_t M, uint32_t N, uint32_t K) {
    const int xr = (es == 4 && M <= 4) ? 4 : M <= 8 ? 8 : 16;
    const uint32_t ksteps = K * es / 256;
    const uint32_t g16 = (N + 15) / 16, g32 = (N + 31) / 32;
    if (xr == 16) return g32 >= 256 ? SklPlan{16, 2, 2, 3} : SklPlan{16, 1, 4, 2};
    if (xr == 8 && es == 2 && ksteps >= 24 && ksteps <= 40 && g32 >= 256 &&
        2 * ((g32 + 255) / 256) <= (g16 + 255) / 256)
        return SklPlan{8, 2, 2, 3};
    if (xr == 8 && ksteps < 64 && g16 >= 512) return SklPlan{8, 1, 2, 2};
    return SklPlan{xr, 1, 4, 2};
}

template <typename T, typename TC, int XR, int S, int R, int WAVES>
void launch_skl(const SkParams& p, hipStream_t st) {
    const uint32_t grid = (p.N + 16 * R - 1) / (16 * R);
    hipLaunchKernelGGL((skinny_lds_kernel<T, TC, XR, S, R, WAVES>), dim3(grid), dim3(64 * WAVES), 0, st, p);
}

template <typename T, typename TC>
int launch_sk_lds(const SkParams& p, hipStream_t st) {
    const SklPlan g = skl_plan(sizeof(T), p.M, p.N, p.K);
    if (g.xr == 16) {
        if (g.r == 2) launch_skl<T, TC, 16, 3, 2, 2>(p, st);
        else launch_skl<T, TC, 16, 2, 1, 4>(p, st);
    } else if (g.xr == 8) {
        if (g.r == 2) launch_skl<T, TC, 8, 3, 2, 2>(p, st);
        else if (g.waves == 2) launch_skl<T, TC, 8, 2, 1, 2>(p, st);
        else launch_skl<T, TC, 8, 2, 1, 4>(p, st);
    } else {
        if constexpr (sizeof(T) == 4) launch_skl<T, TC, 4, 2, 1, 4>(p, st);
    }
    return (int)hipGetLastError();
}

// Staged decode: R weight tiles per wave, MT activation tiles, three stages.
template <typename T, typename TC, int R, int MT>
int launch_dec_lds(const SkParams& p, float* part, int nsplit, hipStream_t st) {
    const dim3 grid((p.N + 64 * R - 1) / (64 * R), (uint32_t)nsplit);
    if (nsplit > 1)
        hipLaunchKernelGGL((decode_lds_kernel<T, float, R, MT, 3, true>), grid, dim3(256), 0, st, p, part, nsplit);
    else
        hipLaunchKernelGGL((decode_lds_kernel<T, TC, R, MT, 3, false>), grid, dim3(256), 0, st, p, part, nsplit);
    return (int)hipGetLastError();
}

template <typename T, typename TC, int R>
int launch_dec_r(const SkParams& p, float* part, int nsplit, hipStream_t st) {
    switch ((p.M + 15) / 16) {
        case 1: return launch_dec_lds<T, TC, R, 1>(p, part, nsplit, st);
        case 2: return launch_dec_lds<T, TC, R, 2>(p, part, nsplit, st);
        case 3: return launch_dec_lds<T, TC, R, 3>(p, part, nsplit, st);
        default: return launch_dec_lds<T, TC, R, 4>(p, part, nsplit, st);
    }
}

template <typename T, typename TC>
int launch_dec_mt(const SkParams& p, float* part, int nsplit, hipStream_t st) {
    return dec_plan(p.N, p.K, sizeof(T)).r == 2 ? launch_dec_r<T, TC, 2>(p, part, nsplit, st)
                                     : launch_dec_r<T, TC, 1>(p, part, nsplit, st);
}

// One element type: output fp32 or the input type.
//   M == 1: the GEMV kernel, 4 weight rows per workgroup (measured best for
//   4096-14336 rows); more activation rows multiply its VALU work and
//   registers.  At M = 2 the staged kernel is ahead (same box, two runs,
//   fp16: 8192^2 23.0 -> 22.0 us, K x O = 4096 x 14336 19.6 -> 18.6,
//   14336 x 4096 20.4 -> 18.8, 4096^2 8.0 -> 7.5; bf16 8192^2 23.2 -> 22.1);
//   at M = 1 it is level or behind (8192^2 22.0 -> 22.3, 4096^2 7.2 -> 7.3,
//   14336 x 4096 19.2 -> 18.7).
//   2 <= M <= DEC_MIN_M - 1: skinny_lds_kernel (skl_plan's geometry).
//   DEC_MIN_M <= M <= 64: decode_lds_kernel, one workgroup per CU, K split
//   nsplit ways over the grid.
template <typename T>
int launch_typed(const SkParams& p, bool f32_out, float* part, int nsplit, hipStream_t st) {
    if (p.M == 1) return f32_out ? launch_gemv<T, float, 1, 4>(p, st) : launch_gemv<T, T, 1, 4>(p, st);
    if ((int)p.M >= DEC_MIN_M)
        return f32_out ? launch_dec_mt<T, float>(p, part, nsplit, st) : launch_dec_mt<T, T>(p, part, nsplit, st);
    return f32_out ? launch_sk_lds<T, float>(p, st) : launch_sk_lds<T, T>(p, st);
}

// skinny_n_kernel K split: slices of whole groups of 4 chunks (64 k), as
// many as keep the grid within 256 workgroups, each slice at least 4
// groups long; SknPlan.per is the chunk count of a slice.
struct SknPlan {
    uint32_t split, per;
};
inline SknPlan skn_plan(uint32_t M, uint32_t N, uint32_t K) {
    const uint32_t cols = M <= 16 ? SKN_COLS : SKN_COLS_MT;
    const uint32_t wg = (N + cols - 1) / cols;
    const uint32_t groups = (K + 63) / 64;
    uint32_t sp = 256 / wg;
    if (sp > groups / 4) sp = groups / 4;
    if (sp > 64) sp = 64;
    if (sp < 1) sp = 1;
    const uint32_t gper = (groups + sp - 1) / sp;
    return SknPlan{(groups + gper - 1) / gper, 4 * gper};
}

template <typename TC, int WV, int MT>
void launch_skn_mt(const SkParams& p, float* part, uint32_t nsplit, int per, hipStream_t st) {
    constexpr int cols = 64 * WV / SKN_KW;
    const dim3 grid((p.N + cols - 1) / cols, nsplit), block(64 * WV);
    if (nsplit > 1)
        hipLaunchKernelGGL((skinny_n_kernel<float, WV, SKN_KW, MT, true>), grid, block, 0, st, p, part, per);
    else
        hipLaunchKernelGGL((skinny_n_kernel<TC, WV, SKN_KW, MT, false>), grid, block, 0, st, p, part, per);
}

// up to 16 rows: eight waves (two column groups of 64); 17-64 rows: four
// waves, one column group, 2-4 activation tiles
template <typename TC>
int launch_skn(const SkParams& p, float* part, uint32_t nsplit, hipStream_t st) {
    const int per = (int)skn_plan(p.M, p.N, p.K).per;
    switch ((p.M + 15) / 16) {
        case 1: launch_skn_mt<TC, SKN_WV, 1>(p, part, nsplit, per, st); break;
        case 2: launch_skn_mt<TC, 4, 2>(p, part, nsplit, per, st); break;
        case 3: launch_skn_mt<TC, 4, 3>(p, part, nsplit, per, st); break;
        default: launch_skn_mt<TC, 4, 4>(p, part, nsplit, per, st); break;
    }
    return (int)hipGetLastError();
}

// skinny_nh_kernel K split: as skn_plan, over workgroups of SKH_COLS
// (M <= 16) or SKH_COLS_MT columns and 32-row chunks (groups of 2 chunks,
// 64 k).
inline SknPlan skh_plan(uint32_t M, uint32_t N, uint32_t K) {
    const uint32_t cols = M <= 16 ? SKH_COLS : SKH_COLS_MT;
    const uint32_t wg = (N + cols - 1) / cols;
    const uint32_t groups = (K + 63) / 64;
    uint32_t sp = 256 / wg;
    if (sp > groups / 4) sp = groups / 4;
    if (sp > 64) sp = 64;
    if (sp < 1) sp = 1;
    const uint32_t gper = (groups + sp - 1) / sp;
    return SknPlan{(groups + gper - 1) / gper, 2 * gper};
}

template <typename T, typename TC, int WV, int MT>
void launch_skh_mt(const SkParams& p, float* part, uint32_t nsplit, int per, hipStream_t st) {
    constexpr int cols = 128 * WV / SKH_KW;
    const dim3 grid((p.N + cols - 1) / cols, nsplit), block(64 * WV);
    if (nsplit > 1)
        hipLaunchKernelGGL((skinny_nh_kernel<T, float, WV, SKH_KW, MT, true>), grid, block, 0, st, p, part, per);
    else
        hipLaunchKernelGGL((skinny_nh_kernel<T, TC, WV, SKH_KW, MT, false>), grid, block, 0, st, p, part, per);
}

template <typename T, typename TC>
int launch_skh(const SkParams& p, float* part, uint32_t nsplit, hipStream_t st) {
    const int per = (int)skh_plan(p.M, p.N, p.K).per;
    switch ((p.M + 15) / 16) {
        case 1: launch_skh_mt<T, TC, SKH_WV, 1>(p, part, nsplit, per, st); break;
        case 2: launch_skh_mt<T, TC, 4, 2>(p, part, nsplit, per, st); break;
        case 3: launch_skh_mt<T, TC, 4, 3>(p, part, nsplit, per, st); break;
        default: launch_skh_mt<T, TC, 4, 4>(p, part, nsplit, per, st); break;
    }
    return (int)hipGetLastError();
}

}  // namespace

extern "C" uint32_t vkb_skinny_plan(int ab_type, int b_kmajor, uint32_t M, uint32_t N, uint32_t K, int64_t lda,
                                   int64_t ldb) {
    if (M == 0 || N == 0 || K == 0 || lda <= 0 || ldb <= 0) return 0;
    const int64_t es = ab_type == VKB_T_F32 ? 4 : 2;
    const int64_t vec = 16 / es;
    if ((M > 1 && (lda % vec || lda < (int64_t)K)) || ldb % vec) return 0;
    if (ab_type == VKB_T_F32) {
        if (!b_kmajor) return (M > 64 || N % 4 || ldb < (int64_t)N) ? 0 : skn_plan(M, N, K).split;
        if (M > 64) return 0;
    } else if (ab_type != VKB_T_F16 && ab_type != VKB_T_BF16) {
        return 0;
    } else if (!b_kmajor) {
        return (M > 64 || N < 8 || N % 8 || ldb < (int64_t)N) ? 0 : skh_plan(M, N, K).split;
    } else if (M > 64) {
        return 0;
    }
    // the staged kernels address a 32-row weight tile and the activation
    // rows (up to 16 ceil(M / 16) of them) with 32-bit buffer offsets: both
    // spans must stay below 2 GiB
    const uint64_t xrows = M <= 16 ? M : 16 * ((M + 15) / 16);
    if (ldb < (int64_t)K || (uint64_t)32 * ldb * es >= (1ull << 31) ||
        ((xrows - 1) * (uint64_t)lda + K) * es >= (1ull << 31))
        return 0;
    if ((int)M < DEC_MIN_M) return 1;
    return dec_plan(N, K, (uint32_t)es).split;
}

extern "C" int vkb_launch_skinny(int ab_type, int b_kmajor, const void* X, int64_t lda, const void* W, int64_t ldb,
                                 void* C, int64_t ldc, int c_type,
                                 uint32_t M, uint32_t N, uint32_t K,
                                 float alpha, float beta, int scalar_mode,
                                 const void* alpha_dev, const void* beta_dev,
                                 const vkb_epilogue_args* epi,
                                 float* part, uint32_t nsplit, void* stream) {
    const uint32_t want = vkb_skinny_plan(ab_type, b_kmajor, M, N, K, lda, ldb);
    if (want == 0 || nsplit != want || (nsplit > 1 && !part)) return (int)hipErrorInvalidValue;
    if (c_type != VKB_T_F32 && c_type != ab_type) return (int)hipErrorInvalidValue;
    if (((uintptr_t)X & 15) || ((uintptr_t)W & 15)) return (int)hipErrorInvalidValue;
    SkParams p{};
    p.X = X; p.W = W; p.C = C;
    p.lda = lda; p.ldb = ldb; p.ldc = ldc;
    p.M = M; p.N = N; p.K = K;
    p.alpha = alpha; p.beta = beta; p.mode = scalar_mode;
    p.alpha_dev = alpha_dev; p.beta_dev = beta_dev;
    // a K split writes raw partials: the reduce applies Cin and bias
    const bool split = nsplit > 1;
    p.epi.cin = (epi && epi->c_in) ? epi->c_in : C;
    p.epi.ldcin = (epi && epi->c_in) ? epi->ldc_in : ldc;
    p.epi.scin = 0;
    p.epi.bias = (epi && !split) ? epi->bias : nullptr;
    p.epi.bias_type = epi ? epi->bias_type : 0;
    hipStream_t st = (hipStream_t)stream;
    const bool f32_out = c_type == VKB_T_F32;
    if (ab_type == VKB_T_F32) {
        if (!b_kmajor) return launch_skn<float>(p, part, nsplit, st);
        if ((int)p.M >= DEC_MIN_M) return launch_dec_mt<float, float>(p, part, (int)nsplit, st);
        return launch_sk_lds<float, float>(p, st);
    }
    if (!b_kmajor) {
        if (ab_type == VKB_T_BF16)
            return f32_out ? launch_skh<__bf16, float>(p, part, nsplit, st) : launch_skh<__bf16, __bf16>(p, part, nsplit, st);
        return f32_out ? launch_skh<_Float16, float>(p, part, nsplit, st)
                       : launch_skh<_Float16, _Float16>(p, part, nsplit, st);
    }
    return ab_type == VKB_T_BF16 ? launch_typed<__bf16>(p, f32_out, part, (int)nsplit, st)
                                 : launch_typed<_Float16>(p, f32_out, part, (int)nsplit, st);
}
