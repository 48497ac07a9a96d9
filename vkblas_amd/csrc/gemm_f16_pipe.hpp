// gemm_f16_pipe.hpp — software-pipelined 256x256x64 fp16 GEMM for gfx950.
//
// Used for full tiles (M, N multiples of 256, K multiple of 128, aligned
// operands); edges and small shapes use gemm_kernel<> in gemm_mfma.hpp, whose
// LDS layout (XOR-swizzled K-contiguous rows) and MFMA role swap this kernel
// shares.  Replaces the reference's large half tiles
// (gemm_half_128x256_bankfree_tmpl.comp, gemm_half_128x128_bankfree_tmpl.comp,
// dispatched from src/vkblas.c:1191-1313).
//
// Per workgroup: 4 waves, 2x2, each owning a 128x128 block of C held in 256
// AGPRs as 4x4 v_mfma_f32_32x32x16_f16 accumulators.  Per 64-wide K step:
//  * K-major operand tiles go global -> LDS directly
//    (global_load_lds_dwordx4: lane l of a wave writes 16 B at M0 + 16 l), so
//    they use no VGPRs and no ds_write.  Each instruction fills eight whole
//    128-byte LDS rows; lane l fetches the global chunk that the XOR swizzle
//    maps to its LDS slot, so the global side stays fully coalesced.
//  * An MN-major operand tile goes through VGPRs: 8x8 fp16 blocks transposed
//    in registers and written K-contiguous (8 ds_write_b128 per lane).
//  * Loads for K step t+1 are issued at the top of step t into the other LDS
//    stage; MFMA fragments for k16 sub-step s+1 are read from LDS while the
//    16 MFMAs of sub-step s run (two register sets).
//  * One barrier per K step.  The K loop is unrolled by two so both LDS
//    stages are compile-time offsets.
//
// LDS map (16-byte units): A stage s at s*2048, B stage s at 4096 + s*2048;
// row r of a tile at r*8, chunk c of row r at slot c ^ g(r), with
// g(r) = r & 7 for K-major tiles (written by whole-row DMA) and
// g(r) = (r ^ (r >> 3)) & 7 for MN-major tiles (written transposed, one row
// per lane 8 rows apart).  Either way 8 consecutive rows read at one chunk hit
// 8 distinct 16-byte bank groups.  A fragment read for k16 sub-step s uses
// chunk 2s + h; because r*8 has its low three bits clear, its slot index is
// (r*8 + (h ^ g(r))) ^ 2s.
//
// Global traffic uses buffer loads on resources based at the tile's first
// element: a fixed per-lane VGPR offset plus a uniform SGPR offset (row step
// and k0), so the loop does no 64-bit address arithmetic.
#pragma once
#include <type_traits>
#include "gemm_mfma.hpp"

namespace vkb {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <typename TC, bool AK, bool BKM>
__global__ __launch_bounds__(256, 1) void gemm_f16_pipe_kernel(KParams p) {
    constexpr int BM = 256, BN = 256, BK = 64;
    constexpr int A0 = 0, B0 = 4096, STG = 2048;   // u32x4 offsets
    __shared__ u32x4 lds[8192];                     // 128 KB

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, h = lane >> 5;

    // ---- tile / batch decode, XCD-aware (as gemm_kernel) ----
    uint32_t bid = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if ((nwg & 7u) == 0) bid = (bid & 7u) * (nwg >> 3) + (bid >> 3);
    const uint32_t per = p.tiles_m * p.tiles_n;
    const uint32_t b = bid / per;
    const uint32_t t = bid - b * per;
    constexpr uint32_t GM = 8;
    const uint32_t width = GM * p.tiles_n;
    const uint32_t group = t / width;
    const uint32_t first_m = group * GM;
    const uint32_t gm = min(p.tiles_m - first_m, GM);
    const uint32_t tin = t - group * width;
    const int m0 = (int)(first_m + tin % gm) * BM;
    const int n0 = (int)(tin / gm) * BN;

    const int lda = (int)p.lda, ldb = (int)p.ldb;
    // Buffer resources on the tile's first element; all per-lane parts are
    // 32-bit byte offsets (the launcher guarantees they fit).
    const _Float16* At = (const _Float16*)p.A + (int64_t)b * p.sa + (AK ? (int64_t)m0 * p.lda : (int64_t)m0);
    const _Float16* Bt = (const _Float16*)p.B + (int64_t)b * p.sb + (BKM ? (int64_t)n0 * p.ldb : (int64_t)n0);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)At, (short)0, -1, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)Bt, (short)0, -1, 0x00020000);
    TC* Cb = (TC*)p.C + (int64_t)b * p.sc;
    const int nkt = (int)(p.K / BK);

    // K-major direct loads: instruction i of this wave fills LDS rows
    // 64 wave + 8 i + [0, 8) (lane -> row + lane / 8, slot lane % 8).  With
    // the K-major swizzle g(r) = r & 7 that slot holds chunk
    // (lane % 8) ^ (lane / 8) for every i, so one VGPR offset serves all
    // eight instructions; the row step 8 i and k0 go in soffset.
    const int koff = ((lane & 7) ^ (lane >> 3)) << 4;
    const int a_voff = (64 * wave + (lane >> 3)) * lda * 2 + koff;
    const int b_voff = (64 * wave + (lane >> 3)) * ldb * 2 + koff;
    // MN-major staged loads: 8x8 block (kb, mb) = (tid / 32, tid % 32)
    const int kb = tid >> 5, mb = tid & 31;
    const int a_mnoff = ((kb * 8) * lda + mb * 8) * 2;
    const int b_mnoff = ((kb * 8) * ldb + mb * 8) * 2;

    u32x4 sa_v[AK ? 1 : 8], sb_v[BKM ? 1 : 8];

    auto issue_loads = [&](int kt, int S) {
        const int k0 = kt * BK;
        // MN-major first, so waiting for them leaves the direct loads in flight
        if constexpr (!AK) {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk)
                sa_v[kk] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_mnoff, (k0 + kk) * lda * 2, 0);
        }
        if constexpr (!BKM) {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk)
                sb_v[kk] = __builtin_amdgcn_raw_buffer_load_b128(rb, b_mnoff, (k0 + kk) * ldb * 2, 0);
        }
        if constexpr (AK) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)&lds[A0 + S * STG + (8 * wave + i) * 64], 16,
                                                         a_voff, k0 * 2 + i * 16 * lda, 0, 0);
        }
        if constexpr (BKM) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)&lds[B0 + S * STG + (8 * wave + i) * 64], 16,
                                                         b_voff, k0 * 2 + i * 16 * ldb, 0, 0);
        }
    };
    // MN-major tiles use the swizzle g(r) = (r ^ (r >> 3)) & 7 (swz), which
    // keeps the transposed writes of 8 lanes (rows 8 apart) on distinct banks
    auto store_staged = [&](int S) {
        if constexpr (!AK) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int r = mb * 8 + i;
                lds[A0 + S * STG + r * 8 + swz(r, kb)] = transpose_row<_Float16>(sa_v, i);
            }
        }
        if constexpr (!BKM) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int r = mb * 8 + i;
                lds[B0 + S * STG + r * 8 + swz(r, kb)] = transpose_row<_Float16>(sb_v, i);
            }
        }
    };

    // fragment slot bases: row * 8 + (h ^ g(row)); sub-step s reads base ^ 2s
    int xa[4], xb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int ra = wm * 128 + i * 32 + l32;
        const int rb = wn * 128 + i * 32 + l32;
        const int ga = AK ? (ra & 7) : ((ra ^ (ra >> 3)) & 7);
        const int gb = BKM ? (rb & 7) : ((rb ^ (rb >> 3)) & 7);
        xa[i] = ra * 8 + (h ^ ga);
        xb[i] = rb * 8 + (h ^ gb);
    }

    floatx16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    u32x4 af[2][4], bf[2][4];
    // Fragment reads are issued one per MFMA pair in the order the next
    // sub-step consumes them: pair q uses A fragment q/2 and B fragments
    // 2(q%2), 2(q%2)+1, so the order is B0 B1 A0 B2 B3 A1 A2 A3.
    auto read_one = [&](int buf, int S, int s, int idx) {
        constexpr int isA[8] = {0, 0, 1, 0, 0, 1, 1, 1};
        constexpr int fi[8] = {0, 1, 0, 2, 3, 1, 2, 3};
        if (isA[idx]) af[buf][fi[idx]] = lds[A0 + S * STG + (xa[fi[idx]] ^ (2 * s))];
        else bf[buf][fi[idx]] = lds[B0 + S * STG + (xb[fi[idx]] ^ (2 * s))];
    };
    auto mfma_pair = [&](int buf, int q) {
        const int i = q >> 1, j = (q & 1) * 2;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, bf[buf][j]),
                                                           __builtin_bit_cast(half8_t, af[buf][i]), acc[i][j], 0, 0, 0);
        acc[i][j + 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            __builtin_bit_cast(half8_t, bf[buf][j + 1]), __builtin_bit_cast(half8_t, af[buf][i]), acc[i][j + 1], 0, 0, 0);
    };

    // Direct (DMA) loads of K step kt+1, one per call (16 per K step: A then B)
    auto dma_one = [&](int kt, int S, int n) {
        const int k0 = (kt + 1) * BK;
        if (n < 8) {
            if constexpr (AK)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)&lds[A0 + (S ^ 1) * STG + (8 * wave + n) * 64],
                                                         16, a_voff, k0 * 2 + n * 16 * lda, 0, 0);
        } else {
            if constexpr (BKM)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)&lds[B0 + (S ^ 1) * STG + (8 * wave + n - 8) * 64],
                                                         16, b_voff, k0 * 2 + (n - 8) * 16 * ldb, 0, 0);
        }
    };
    // MN-major staged loads of K step kt (one k row per call, 8 per operand)
    auto stage_load = [&](int kt, int kk) {
        const int k0 = kt * BK;
        if constexpr (!AK) sa_v[kk] = __builtin_amdgcn_raw_buffer_load_b128(ra, a_mnoff, (k0 + kk) * lda * 2, 0);
        if constexpr (!BKM) sb_v[kk] = __builtin_amdgcn_raw_buffer_load_b128(rb, b_mnoff, (k0 + kk) * ldb * 2, 0);
    };
    auto stage_store = [&](int S, int i) {
        const int r = mb * 8 + i;
        if constexpr (!AK) lds[A0 + S * STG + r * 8 + swz(r, kb)] = transpose_row<_Float16>(sa_v, i);
        if constexpr (!BKM) lds[B0 + S * STG + r * 8 + swz(r, kb)] = transpose_row<_Float16>(sb_v, i);
    };
    constexpr bool STAGED = !AK || !BKM;

    // Region between two barriers, stage S = K step kt:
    //   sub-step 3 of K step kt-1 (buf 1)  + reads of (kt, sub-step 0) -> buf 0,
    //                                        DMA of kt+1 -> stage S^1
    //   sub-step 0 of kt (buf 0)           + reads of sub-step 1 -> buf 1
    //   sub-step 1 of kt (buf 1)           + reads of sub-step 2 -> buf 0,
    //                                        staged rows of kt+1 -> LDS stage S^1
    //   sub-step 2 of kt (buf 0)           + reads of sub-step 3 -> buf 1,
    //                                        staged loads of kt+2 -> VGPRs
    //   wait for this wave's loads and LDS traffic, barrier
    // Every unit (MFMA pair + its companions) is fenced with sched_barrier
    // so the compiler keeps this order and both fragment sets live.
    auto region = [&](int kt, int S, bool prev, bool next, bool next2) {
        // The DMA of step kt+1 starts right after the barrier: stage S^1 was
        // last read before it, and the loads get four sub-steps to land.
        if (prev) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                mfma_pair(1, q);
                read_one(0, S, 0, q);
                if (next) {
                    dma_one(kt, S, 2 * q);
                    dma_one(kt, S, 2 * q + 1);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            mfma_pair(0, q);
            read_one(1, S, 1, q);
            if (next && !prev) {
                dma_one(kt, S, 2 * q);
                dma_one(kt, S, 2 * q + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            mfma_pair(1, q);
            read_one(0, S, 2, q);
            if (STAGED && next) stage_store(S ^ 1, q);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            mfma_pair(0, q);
            read_one(1, S, 3, q);
            if (STAGED && next2) stage_load(kt + 2, q);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };

    // ---- prologue: K step 0 into stage 0 (and staged rows of step 1) ----
    issue_loads(0, 0);
    store_staged(0);
    if constexpr (STAGED) {
        if (nkt > 1) {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) stage_load(1, kk);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 8; ++q) read_one(0, 0, 0, q);

    // nkt is even (K % 128 == 0): regions alternate stages 0 and 1; the
    // loop body is branch-free, the last two regions load less
    if (nkt == 2) {
        region(0, 0, false, true, false);
        region(1, 1, true, false, false);
    } else {
        region(0, 0, false, true, true);
        int kt = 1;
        for (; kt + 3 < nkt; kt += 2) {
            region(kt, 1, true, true, true);
            region(kt + 1, 0, true, true, true);
        }
        region(kt, 1, true, true, true);       // kt == nkt - 3: stages step nkt-1
        region(kt + 1, 0, true, true, false);  // loads step nkt-1
        region(kt + 2, 1, true, false, false);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) mfma_pair(1, q);   // sub-step 3 of the last K step

    // ---- epilogue: C[m][n..n+3] = alpha * acc + beta * C ----
    float alpha, beta;
    load_scalars(p, alpha, beta);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + wm * 128 + i * 32 + l32;
        TC* crow = Cb + (int64_t)m * p.ldc;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wn * 128 + j * 32 + q * 8 + h * 4;
                float x[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) x[e] = alpha * acc[i][j][q * 4 + e];
                if (beta != 0.0f) {
                    float o[4];
                    load4<TC>(crow + n, o, true);
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[e] += beta * o[e];
                }
                store4<TC>(crow + n, x, true);
            }
        }
    }
}

}  // namespace vkb
