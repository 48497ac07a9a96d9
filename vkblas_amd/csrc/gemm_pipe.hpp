// gemm_pipe.hpp — software-pipelined 256x256 GEMM for gfx950, fp16 and fp32.
//
// Used for full tiles (M, N multiples of 256, K a multiple of two K steps,
// aligned operands); edges and small shapes use gemm_kernel<> in
// gemm_mfma.hpp, whose MFMA role swap and epilogue this kernel shares.
// Replaces the reference's large tiles (gemm_f32_128x128_bankfree_tmpl.comp,
// gemm_half_128x256_bankfree_tmpl.comp, gemm_half_128x128_bankfree_tmpl.comp,
// dispatched from src/vkblas.c:1191-1313, 1822-1868).
//
// Per workgroup: 4 waves, 2x2, each owning a 128x128 block of C held in 256
// AGPRs as 4x4 32x32 MFMA accumulators.  A K step is 128 bytes of K (64 fp16
// or 32 fp32) and four sub-steps of one 16-byte chunk per lane half:
//  * fp16: sub-step s = v_mfma_f32_32x32x16_f16 over chunk 2s + h, 16 MFMAs;
//  * fp32: sub-step s = v_mfma_f32_32x32x2_f32 over chunk 4h + s, one MFMA per
//    k of the chunk, 64 MFMAs.
// Per K step:
//  * K-major operand tiles go global -> LDS directly (buffer_load ... lds:
//    lane l of a wave writes 16 B at M0 + 16 l), so they use no VGPRs and no
//    ds_write.  Each instruction fills eight whole 128-byte LDS rows; lane l
//    fetches the global chunk that the swizzle maps to its LDS slot, so the
//    global side stays fully coalesced.
//  * An MN-major operand tile goes through VGPRs: VEC x VEC blocks
//    transposed in registers and written K-contiguous (8 ds_write_b128 per
//    lane).
//  * Loads for K step t+1 are issued during step t into the other LDS stage;
//    MFMA fragments for sub-step s+1 are read from LDS while the MFMAs of
//    sub-step s run (two register sets).
//  * One barrier per K step.  The K loop is unrolled by two so both LDS
//    stages are compile-time offsets.
//
// LDS map (16-byte units): A stage s at s*2304, B stage s at 4608 + s*2304
// (144 KB).  gfx950's LDS is 64 banks (256 bytes) wide and serves a
// ds_read_b128 16 lanes at a time, so the 16 rows a fragment read touches at
// one chunk must land on 16 distinct 16-byte bank groups: the 8 rows of one
// row parity share a 256-byte bank line half and need 8 distinct slots.
//  * MN-major tiles (written transposed through VGPRs): row r at r*8, chunk c
//    at slot c ^ g(r), g(r) = (r ^ (r >> 3)) & 7 — over 16 consecutive rows
//    each parity class sees all 8 slots.
//  * K-major tiles (written by whole-row DMA, lane l -> +16 l, so the swizzle
//    can only depend on r & 7): rows come in groups of 8 at a 1152-byte
//    stride (72 units, 128 bytes of padding per group), row r at
//    (r >> 3)*72 + (r & 7)*8, chunk c at slot c ^ (r & 7).  The padding
//    moves odd groups to the other half of the bank line, which separates
//    rows r and r + 8 that share r & 7.
// Every row base has its low three bits clear, so a fragment's slot index is
// (base + (hoff ^ g)) ^ sub-step offset (2s for fp16, s for fp32).
//
// Global traffic uses buffer loads on resources based at the tile's first
// element: a fixed per-lane VGPR offset plus a uniform SGPR offset (row step
// and k0), so the loop does no 64-bit address arithmetic.
#pragma once
#include <type_traits>
#include "gemm_mfma.hpp"

namespace vkb {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

#ifndef VKB_PIPE_DMA_UNITS
#define VKB_PIPE_DMA_UNITS 16
#endif

template <typename T, typename TC, bool AK, bool BKM>
__global__ __launch_bounds__(256, 1) void gemm_pipe_kernel(KParams p) {
    constexpr bool F16 = sizeof(T) == 2;
    constexpr int ES = sizeof(T);                   // element bytes
    constexpr int BM = 256, BN = 256, BK = 128 / ES;
    constexpr int VEC = 16 / ES;                    // elements per 16-byte chunk
    constexpr int A0 = 0, B0 = 4608, STG = 2304;    // u32x4 offsets
    constexpr int GRP = 72;                         // 8-row group stride of K-major tiles
    __shared__ u32x4 lds[9216];                     // 144 KB

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
    const T* At = (const T*)p.A + (int64_t)b * p.sa + (AK ? (int64_t)m0 * p.lda : (int64_t)m0);
    const T* Bt = (const T*)p.B + (int64_t)b * p.sb + (BKM ? (int64_t)n0 * p.ldb : (int64_t)n0);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)At, (short)0, -1, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)Bt, (short)0, -1, 0x00020000);
    TC* Cb = (TC*)p.C + (int64_t)b * p.sc;
    const int nkt = (int)(p.K / BK);

    // K-major direct loads: instruction i of this wave fills the 8-row group
    // 8 wave + i (rows 64 wave + 8 i + [0, 8); lane -> row + lane / 8, slot
    // lane % 8).  With the K-major swizzle c ^ (r & 7) that slot holds chunk
    // (lane % 8) ^ (lane / 8) for every i, so one VGPR offset serves all
    // eight instructions; the row step 8 i and k0 go in soffset.
    const int koff = ((lane & 7) ^ (lane >> 3)) << 4;
    const int a_voff = (64 * wave + (lane >> 3)) * lda * ES + koff;
    const int b_voff = (64 * wave + (lane >> 3)) * ldb * ES + koff;
    // MN-major staged loads: VECxVEC blocks (kb, mb + 32 blk), kb = tid / 32
    // (k rows kb*VEC..), mb = tid % 32 (columns (mb + 32 blk)*VEC..)
    const int kb = tid >> 5, mb = tid & 31;
    auto mn_off = [&](int ld, int blk) { return ((kb * VEC) * ld + (mb + 32 * blk) * VEC) * ES; };

    // Barrier after "s_waitcnt vmcnt(n) lgkmcnt(0)": the staged loads issued
    // after a K step's DMA may stay in flight; vector loads complete in issue
    // order, so this still waits for the DMA.  The barrier is written out
    // (no __syncthreads) because its workgroup fence would wait for every
    // outstanding load; the "memory" clobber keeps the compiler from moving
    // LDS accesses across it.
    constexpr int NSTAGED = (AK ? 0 : 8) + (BKM ? 0 : 8);
    auto sync_vm = [](auto n_c) {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(decltype(n_c)::value) : "memory");
    };

    // staged registers: index blk * VEC + k row within the block
    u32x4 sa_v[AK ? 1 : 8], sb_v[BKM ? 1 : 8];

    // Direct (DMA) load n of K step kt (8 per operand per wave: A then B)
    auto dma_load = [&](int kt, int S, int n) {
        const int k0 = kt * BK;
        if (n < 8) {
            if constexpr (AK)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)&lds[A0 + S * STG + (8 * wave + n) * GRP], 16,
                                                         a_voff, (k0 + n * 8 * lda) * ES, 0, 0);
        } else {
            if constexpr (BKM)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)&lds[B0 + S * STG + (8 * wave + n - 8) * GRP],
                                                         16, b_voff, (k0 + (n - 8) * 8 * ldb) * ES, 0, 0);
        }
    };
    // MN-major staged load v of K step kt (8 per operand)
    auto stage_load = [&](int kt, int v) {
        const int k0 = kt * BK + (v % VEC);
        const int blk = v / VEC;
        if constexpr (!AK) sa_v[v] = __builtin_amdgcn_raw_buffer_load_b128(ra, mn_off(lda, blk), k0 * lda * ES, 0);
        if constexpr (!BKM) sb_v[v] = __builtin_amdgcn_raw_buffer_load_b128(rb, mn_off(ldb, blk), k0 * ldb * ES, 0);
    };
    // MN-major tiles use the swizzle g(r) = (r ^ (r >> 3)) & 7 (swz), which
    // keeps the transposed writes of lanes on distinct banks.  Row v of the
    // thread's blocks: block v / VEC, row (mb + 32 blk)*VEC + v % VEC.
    auto stage_store = [&](int S, int v) {
        const int blk = v / VEC, i = v % VEC;
        const int r = (mb + 32 * blk) * VEC + i;
        if constexpr (!AK) lds[A0 + S * STG + r * 8 + swz(r, kb)] = transpose_row<T>(&sa_v[blk * VEC], i);
        if constexpr (!BKM) lds[B0 + S * STG + r * 8 + swz(r, kb)] = transpose_row<T>(&sb_v[blk * VEC], i);
    };
    constexpr bool STAGED = !AK || !BKM;

    // fragment slot bases: row base + (hoff ^ g(row)); sub-step s reads
    // base ^ (s * SX)
    constexpr int SX = F16 ? 2 : 1;
    const int hoff = F16 ? h : 4 * h;
    auto frag_base = [&](int r, bool kmajor) {
        return kmajor ? (r >> 3) * GRP + (r & 7) * 8 + (hoff ^ (r & 7)) : r * 8 + (hoff ^ ((r ^ (r >> 3)) & 7));
    };
    int xa[4], xb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        xa[i] = frag_base(wm * 128 + i * 32 + l32, AK);
        xb[i] = frag_base(wn * 128 + i * 32 + l32, BKM);
    }

    floatx16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    u32x4 af[2][4], bf[2][4];
    // A sub-step is 8 units (one fragment read of the next sub-step each).
    // fp16: unit q = MFMAs of tiles (q/2, 2(q%2)) and (q/2, 2(q%2)+1), so the
    //   next sub-step's fragments are read in the order B0 B1 A0 B2 B3 A1 A2 A3.
    // fp32: unit q = k element q/2 of the chunk on the 8 tiles of half q%2
    //   (rows i = 2(q%2), 2(q%2)+1), reads in the order B0..B3 A0..A3.
    auto read_one = [&](int buf, int S, int s, int idx) {
        constexpr int isA16[8] = {0, 0, 1, 0, 0, 1, 1, 1};
        constexpr int fi16[8] = {0, 1, 0, 2, 3, 1, 2, 3};
        const bool isA = F16 ? isA16[idx] : idx >= 4;
        const int fi = F16 ? fi16[idx] : (idx & 3);
        if (isA) af[buf][fi] = lds[A0 + S * STG + (xa[fi] ^ (SX * s))];
        else bf[buf][fi] = lds[B0 + S * STG + (xb[fi] ^ (SX * s))];
    };
    auto mfma_unit = [&](int buf, int q) {
        if constexpr (F16) {
            const int i = q >> 1, j = (q & 1) * 2;
#pragma unroll
            for (int jj = j; jj < j + 2; ++jj)
                acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, bf[buf][jj]),
                                                                    __builtin_bit_cast(half8_t, af[buf][i]),
                                                                    acc[i][jj], 0, 0, 0);
        } else {
            const int e = q >> 1, i0 = (q & 1) * 2;
#pragma unroll
            for (int i = i0; i < i0 + 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(bf[buf][j][e]),
                                                                    __uint_as_float(af[buf][i][e]), acc[i][j], 0, 0, 0);
        }
    };

    // The 16 DMA loads of a K step are spread over DMA_UNITS consecutive
    // units from the region's first: issued in a burst they oversubscribe the
    // texture address unit and stall the MFMA issue.
    constexpr int DMA_UNITS = VKB_PIPE_DMA_UNITS;
    // the first region's DMA starts at unit 8 and must end before the staged
    // loads of unit 24 (the end-of-region wait counts on that order)
    static_assert(DMA_UNITS >= 1 && DMA_UNITS <= 16, "DMA must precede the staged loads");
    auto dma_unit = [&](int kt, int S, int v) {   // v: unit index from the first
#pragma unroll
        for (int n = 0; n < 16; ++n)
            if (n * DMA_UNITS >= v * 16 && n * DMA_UNITS < (v + 1) * 16) dma_load(kt, S, n);
    };

    // Region between two barriers, stage S = K step kt:
    //   sub-step 3 of K step kt-1 (buf 1)  + reads of (kt, sub-step 0) -> buf 0
    //   sub-step 0 of kt (buf 0)           + reads of sub-step 1 -> buf 1
    //   sub-step 1 of kt (buf 1)           + reads of sub-step 2 -> buf 0,
    //                                        staged rows of kt+1 -> LDS stage S^1
    //   sub-step 2 of kt (buf 0)           + reads of sub-step 3 -> buf 1,
    //                                        staged loads of kt+2 -> VGPRs
    //   the DMA of kt+1 -> stage S^1 spread over the first DMA_UNITS units
    //   wait for this wave's DMA and LDS traffic, barrier
    // Every unit (MFMAs + companions) is fenced with sched_barrier so the
    // compiler keeps this order and both fragment sets live.
    auto region = [&](int kt, int S, bool prev, bool next, bool next2) {
        // stage S^1 was last read before the barrier that opened this region
        const int u0 = prev ? 0 : 8;   // first unit of this region
        if (prev) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                mfma_unit(1, q);
                read_one(0, S, 0, q);
                if (next) dma_unit(kt + 1, S ^ 1, q - u0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            mfma_unit(0, q);
            read_one(1, S, 1, q);
            if (next) dma_unit(kt + 1, S ^ 1, 8 + q - u0);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            mfma_unit(1, q);
            read_one(0, S, 2, q);
            if (next) dma_unit(kt + 1, S ^ 1, 16 + q - u0);
            if (STAGED && next) stage_store(S ^ 1, q);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            mfma_unit(0, q);
            read_one(1, S, 3, q);
            if (next) dma_unit(kt + 1, S ^ 1, 24 + q - u0);
            if (STAGED && next2) stage_load(kt + 2, q);
            __builtin_amdgcn_sched_barrier(0);
        }
        // DMA of kt+1 landed (staged loads of kt+2 may still fly)
        if (next && next2) sync_vm(std::integral_constant<int, NSTAGED>{});
        else sync_vm(std::integral_constant<int, 0>{});
    };

    // ---- prologue: K step 0 into stage 0 (and staged rows of step 1) ----
    if constexpr (STAGED) {
        // MN-major first, so waiting for them leaves the direct loads in flight
#pragma unroll
        for (int v = 0; v < 8; ++v) stage_load(0, v);
    }
#pragma unroll
    for (int n = 0; n < 16; ++n) dma_load(0, 0, n);
    if constexpr (STAGED) {
#pragma unroll
        for (int v = 0; v < 8; ++v) stage_store(0, v);
#pragma unroll
        for (int v = 0; v < 8; ++v) stage_load(1, v);   // nkt >= 2
    }
    sync_vm(std::integral_constant<int, NSTAGED>{});
#pragma unroll
    for (int q = 0; q < 8; ++q) read_one(0, 0, 0, q);

    // nkt is even: regions alternate stages 0 and 1; the loop body is
    // branch-free, the last two regions load less
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
    for (int q = 0; q < 8; ++q) mfma_unit(1, q);   // sub-step 3 of the last K step

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
