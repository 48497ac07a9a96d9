// gemm_wavek.hpp — split-K pass 1 on small output tiles (32x32 or 64x64),
// the workgroup's K slice divided among its four waves.
//
// For a split-K GEMM with few output tiles (M = N = 256 with a caller's split
// of 4 or 16: 64 or 16 tiles of 32x32 / 64x64 per K slice, 256 workgroups in
// all) the tile kernels either leave most CUs idle (128x128 tiles: 16 or 64
// workgroups) or run their 2x2 wave grid on 16x16 / 32x32 wave tiles with a
// barrier every few MFMAs.  Here every wave of a workgroup computes the
// whole TT x TT tile over a quarter of the slice's K steps:
//  * no barrier in the K loop: a wave copies its own operand steps into its
//    own LDS stages (buffer_load ... lds, lane l writes 16 B at M0 + 16 l)
//    and waits for them with s_waitcnt vmcnt, S stages deep;
//  * fragments are read from LDS as in gemm_pipe.hpp: ds_read_b128 of
//    K-major rows, ds_read_b64_tr_b16 of 16-bit MN-major rows, ds_read_b32
//    of fp32 MN-major rows, each layout swizzled so a read touches every
//    16-byte bank group once;
//  * at the end the four waves' sums meet in LDS and are added in wave
//    order (0 + 1, + 2, + 3: a fixed order, so the partials are bitwise
//    reproducible) and written as the slice's raw fp32 partial, which the
//    fixed-order reduce (splitk_reduce.hip) sums over the slices.
// Replaces the reference's split-K pass 1 for small outputs
// (gemm_f32_64x64_splitk_tmpl.comp, gemm_half_128x128_splitk_tmpl.comp,
// dispatched from src/vkblas.c:1873-1984, 1990-2096).
//
// A K step is 32 k of fp32 (128 bytes) and 32 or 64 k of fp16 / bf16 (64 or
// 128 bytes).  MFMAs, with the roles swapped as everywhere here (src A = B
// fragment, src B = A fragment, so a lane holds 4 consecutive n of one row m):
//  * 16-bit: v_mfma_f32_16x16x32 on (TT/16)^2 tiles, one per tile and 32-k
//    sub-step (lane group g = lane / 16 holds k 8g .. 8g+7 of row lane % 16);
//  * fp32: v_mfma_f32_32x32x2_f32 on (TT/32)^2 tiles, four sub-steps of 8 k,
//    lane half h holding k 8s + 4h .. +3 of its row and MFMA e taking
//    element e.
//
// LDS, per wave, per stage, per operand (16-byte units, u):
//  * 16-bit K-major, 64-byte rows: row r (of TT) at 4r, chunk c (8 k) at slot
//    c ^ ((r >> 2) & 3).  The 16 lanes of a lane group read rows q = 0..15 at
//    one chunk: bank group 4 (q & 3) + (c ^ (q >> 2)) takes 16 distinct
//    values.  128-byte rows: row r at 8r, chunk c at c ^ (r & 7), as the
//    pipelined kernel's 16-bit K-major tiles.
//  * 16-bit MN-major: k row k (of 32 or 64) at k CPR (CPR = TT / 8 chunks of 8
//    columns), chunk c at slot c ^ t(k); TT 64: t = 2 (k >> 1 & 1) + 4 (k >>
//    3 & 1), TT 32: t = 2 (k >> 3 & 1).  A 32-lane half of a transposing read
//    touches the rows 8g + 0..3 of two lane groups at two chunks 2f, 2f + 1:
//    with the row's bank offset (CPR k mod 16) t separates every pair of rows
//    that share it, so the 16 chunks fall on 16 bank groups.  t(k + 4) =
//    t(k + 32) = t(k): the second read of a fragment and the second sub-step
//    are immediate offsets.
//  * fp32 K-major: row r at (r >> 3) 72 + (r & 7) 8, chunk c at c ^ (r & 7)
//    (the 1152-byte group stride separates rows r and r + 8, which a 32-row
//    fragment read also touches).
//  * fp32 MN-major, TT 64: k row k at 16k, chunk c at c ^ 8 (k >> 2 & 1); a
//    read has lanes 0-31 on row k and lanes 32-63 on row k + 4, which then
//    take opposite halves of the 64 banks.  TT 32: k row k at 8 p(k), p(k) =
//    k ^ (k >> 2 & 1), so rows k and k + 4 sit on rows of opposite parity.
#pragma once
#include "gemm_pipe.hpp"

namespace vkb {

// KB16: bytes of K per step for 16-bit types (64: 32 k, one sub-step; 128:
// 64 k, two sub-steps and whole 128-byte rows of a K-major operand); fp32
// always 128 (32 k, four sub-steps).  Stages: as many as fit in 144 KB (at
// most 8).
template <typename T, int TT, int KB16>
struct WaveKGeom {
    static constexpr bool F16 = sizeof(T) == 2;
    static constexpr int ES = sizeof(T);
    static constexpr int KS = F16 ? KB16 / 2 : 32;               // k per step
    static constexpr int NSUB = F16 ? KS / 32 : 4;               // MFMA sub-steps per step
    static constexpr int OPU = F16 ? KB16 * TT / 16 : (TT / 8) * 72;   // units per operand per stage
    static constexpr int STU = 2 * OPU;                          // units per stage
    static constexpr int S = (9216 / 4) / STU > 8 ? 8 : (9216 / 4) / STU;   // stages per wave
    static constexpr int WU = S * STU;                           // units per wave
    static constexpr int NDO = OPU / (F16 ? 64 : 72);            // DMA instructions per operand and step
    static constexpr int ND = 2 * NDO;
};

// Workgroups per (slice, tile) when a launch divides each K slice (KParams
// nq > 1; the launcher passes 1 or this).
constexpr int WAVEK_NQ = 4;

template <typename T, bool AK, bool BKM, int TT, int KB16 = 64>
__global__ __launch_bounds__(256, 1) void gemm_wavek_kernel(KParams p) {
    using G = WaveKGeom<T, TT, KB16>;
    constexpr bool F16 = G::F16;
    constexpr int ES = G::ES, KS = G::KS, NSUB = G::NSUB, OPU = G::OPU, STU = G::STU, S = G::S, WU = G::WU;
    constexpr int NDO = G::NDO, ND = G::ND;
    static_assert(TT == 32 || TT == 64, "32x32 or 64x64 tiles");
    static_assert(KB16 == 64 || KB16 == 128, "16-bit K step of 32 or 64 k");
    static_assert(S >= 2 && S <= 8 && (S - 1) * ND <= 63, "stage count / vmcnt range");
    __shared__ u32x4 lds[4 * WU];   // 144 KB

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int q = lane & 15, g = lane >> 4;

    // ---- tile and slice, XCD-aware (the tiles of a slice share an XCD) ----
    uint32_t bid = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if ((nwg & 7u) == 0) bid = (bid & 7u) * (nwg >> 3) + (bid >> 3);
    const uint32_t per = p.tiles_m * p.tiles_n;
    const uint32_t nq = p.nq > 1 ? WAVEK_NQ : 1;  // workgroups per (slice, tile)
    const uint32_t bq = bid / per;                // slice b, part q: bq = b nq + q
    const uint32_t t = bid - bq * per;
    const uint32_t b = bq / nq, qi = bq - b * nq;
    const int m0 = (int)(t / p.tiles_n) * TT, n0 = (int)(t % p.tiles_n) * TT;
    // slice b: k in [b kps, min(K, (b + 1) kps)), nsl steps; part q takes
    // steps [nsl q / nq, nsl (q + 1) / nq) of them, ns in all, and wave w
    // the steps [ns w / 4, ns (w + 1) / 4) of those
    const int64_t kbeg = (int64_t)b * p.kps;
    const uint32_t klen = min(p.K - (uint32_t)kbeg, p.kps);
    const int nsl = (int)(klen / KS);
    const int qs0 = (int)(((uint32_t)nsl * qi) / nq);
    const int ns = (int)(((uint32_t)nsl * (qi + 1)) / nq) - qs0;
    const int s0 = qs0 + ((ns * wave) >> 2), n = ((ns * (wave + 1)) >> 2) - ((ns * wave) >> 2);
    const int64_t kw = kbeg + (int64_t)s0 * KS;
    const int lda = (int)p.lda, ldb = (int)p.ldb;
    const T* At = (const T*)p.A + (AK ? (int64_t)m0 * p.lda + kw : kw * p.lda + m0);
    const T* Bt = (const T*)p.B + (BKM ? (int64_t)n0 * p.ldb + kw : kw * p.ldb + n0);
    auto rsrc_words = [](const void* base) {
        const uint64_t a = (uint64_t)base;
        return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                     __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32) & 0xffff), -1, 0x00020000};
    };
    const i32x4 ra = rsrc_words(At), rb = rsrc_words(Bt);
    const int wbase = wave * WU;   // this wave's LDS units

    // ---- DMA: per-lane byte offsets (the instruction's row step and the
    // step's k go in soffset) ----
    // K-major, 16-bit, 64-byte rows: instruction i covers rows 16i .. 16i+15
    // (lane -> row lane / 4, slot lane % 4, which holds chunk (lane % 4) ^
    // (lane >> 4 & 3)).
    // K-major, fp32 and 16-bit with 128-byte rows: rows 8i .. 8i+7 (lane ->
    // row lane / 8, slot lane % 8, chunk (lane % 8) ^ (lane / 8)), written at
    // the group base 72 i (fp32) or 64 i.
    // MN-major, 16-bit: RPB = 64 / CPR k rows per instruction (lane -> row
    // lane / CPR, slot lane % CPR, chunk slot ^ t(row)); TT 64: t depends on
    // the instruction through i & 1.
    // MN-major, fp32, TT 64: rows 4i .. 4i+3 (lane -> row lane / 16, slot
    // lane % 16, chunk slot ^ 8 (i & 1)); TT 32: physical rows 8i .. 8i+7
    // (lane -> physical row lane / 8 = k row (lane / 8) ^ (lane >> 5), chunk
    // lane % 8).
    constexpr int CPR = TT / 8, RPB = 64 / CPR;
    auto tk16 = [](int k) { return TT == 64 ? 2 * ((k >> 1) & 1) + 4 * ((k >> 3) & 1) : 2 * ((k >> 3) & 1); };
    auto dma_voff = [&](bool kmaj, int ld, int var) -> int {
        if (kmaj) {
            if constexpr (F16 && KB16 == 64) return (lane >> 2) * ld * ES + (((lane & 3) ^ ((lane >> 4) & 3)) << 4);
            else return (lane >> 3) * ld * ES + (((lane & 7) ^ (lane >> 3)) << 4);
        }
        if constexpr (F16) {
            const int r = RPB * var + lane / CPR;   // var: an instruction with this i & 1
            return (lane / CPR) * ld * ES + (((lane % CPR) ^ tk16(r)) << 4);
        } else if constexpr (TT == 64) {
            return (lane >> 4) * ld * ES + (((lane & 15) ^ (8 * var)) << 4);
        } else {
            return ((lane >> 3) ^ (lane >> 5)) * ld * ES + ((lane & 7) << 4);
        }
    };
    const int av0 = dma_voff(AK, lda, 0), av1 = dma_voff(AK, lda, 1);
    const int bv0 = dma_voff(BKM, ldb, 0), bv1 = dma_voff(BKM, ldb, 1);
    auto dma = [&](const i32x4& rs, int dst_unit, int voff, int soff) {
        const int m0r = __builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(lds_ptr_t)&lds[dst_unit]);
        asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
                     :: "v"(voff), "s"(rs), "s"(__builtin_amdgcn_readfirstlane(soff)), "{m0}"(m0r)
                     : "memory");
    };
    // instruction i of one operand of step j into stage st
    auto dma_op = [&](bool isA, int j, int st, int i) {
        const bool kmaj = isA ? AK : BKM;
        const int ld = isA ? lda : ldb;
        const int v = (i & 1) ? (isA ? av1 : bv1) : (isA ? av0 : bv0);
        const int base = wbase + st * STU + (isA ? 0 : OPU);
        int dst, soff;
        if (kmaj) {
            dst = base + (F16 ? 64 * i : 72 * i);
            soff = (j * KS + (F16 && KB16 == 64 ? 16 : 8) * i * ld) * ES;
        } else if constexpr (F16) {
            dst = base + 64 * i;
            soff = (j * KS + RPB * i) * ld * ES;
        } else {
            dst = base + 64 * i;
            soff = (j * KS + (TT == 64 ? 4 : 8) * i) * ld * ES;
        }
        dma(isA ? ra : rb, dst, v, soff);
    };
    auto dma_step = [&](int j, int st) {
#pragma unroll
        for (int i = 0; i < NDO; ++i) {
            dma_op(true, j, st, i);
            dma_op(false, j, st, i);
        }
    };
    // s_waitcnt vmcnt(c * ND): the DMA of the c steps issued after the one
    // waited for may stay in flight (vector memory completes in order)
    auto wait_steps = [](int c) {
        switch (c) {
            case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
            case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(1 * G::ND) : "memory"); break;
            case 2: if constexpr (S > 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * G::ND) : "memory"); break;
            case 3: if constexpr (S > 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * G::ND) : "memory"); break;
            case 4: if constexpr (S > 4) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * G::ND) : "memory"); break;
            case 5: if constexpr (S > 5) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(5 * G::ND) : "memory"); break;
            default: if constexpr (S > 6) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(6 * G::ND) : "memory"); break;
        }
    };

    // ---- fragments ----
    constexpr int NF = F16 ? TT / 16 : TT / 32;     // fragments per operand
    // per-lane byte bases within a stage operand
    int kb16[2] = {};        // 16-bit K-major, per sub-step: row q, chunk 4s + g
    int kb32[4] = {};        // fp32 K-major, per sub-step: row l32, chunk 2s + h
    int tb16[NF] = {};       // 16-bit MN-major, per fragment
    int mb32[4] = {};        // fp32 MN-major (TT 64: per fragment; TT 32: per element)
    if constexpr (F16) {
        if constexpr (KB16 == 64) {
            kb16[0] = (4 * q + (g ^ ((q >> 2) & 3))) * 16;
        } else {
#pragma unroll
            for (int s = 0; s < 2; ++s) kb16[s] = (8 * q + ((4 * s + g) ^ (q & 7))) * 16;
        }
        const int tk = TT == 64 ? 2 * ((q >> 3) & 1) + 4 * (g & 1) : 2 * (g & 1);
#pragma unroll
        for (int f = 0; f < NF; ++f)
            tb16[f] = ((8 * g + (q >> 2)) * CPR + (((2 * f) ^ tk) + ((q >> 1) & 1))) * 16 + 8 * (q & 1);
    } else {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            kb32[s] = ((l32 >> 3) * 72 + (l32 & 7) * 8 + ((2 * s) ^ h ^ (l32 & 7))) * 16;
        if constexpr (TT == 64) {
#pragma unroll
            for (int f = 0; f < 2; ++f) mb32[f] = 1024 * h + 128 * (f ^ h) + 4 * l32;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) mb32[e] = (4 * h + (e ^ h)) * 128 + 4 * l32;
        }
    }
    auto tr_read = [&](int byte_off) {
        const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)((char*)lds + byte_off));
        return __builtin_bit_cast(u32x2, v);
    };
    // fragment f of one operand of stage st, sub-step s
    auto frag = [&](bool isA, int st, int s, int f) -> u32x4 {
        const bool kmaj = isA ? AK : BKM;
        const int ob = (wbase + st * STU + (isA ? 0 : OPU)) * 16;   // bytes
        if constexpr (F16) {
            if (kmaj) return *(const u32x4*)((const char*)lds + ob + kb16[s] + (KB16 / 16) * 16 * 16 * f);
            const u32x2 lo = tr_read(ob + tb16[f] + 32 * s * CPR * 16);
            const u32x2 hi = tr_read(ob + tb16[f] + (32 * s + 4) * CPR * 16);
            return u32x4{lo[0], lo[1], hi[0], hi[1]};
        } else {
            if (kmaj) return *(const u32x4*)((const char*)lds + ob + kb32[s] + 288 * 16 * f);
            u32x4 r;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int off = TT == 64 ? mb32[f] + (8 * s + e) * 256 : mb32[e] + 8 * s * 128;
                r[e] = *(lds_u32_t*)((const char*)lds + ob + off);
            }
            return r;
        }
    };

    // Accumulators: NC copies of the tile's NF x NF accumulator tiles, so
    // that consecutive MFMAs never feed each other (a dependent MFMA waits
    // for its predecessor's result): fp32 32x32 tiles (one tile) take four
    // copies, the MFMA of element e going to copy e; every other shape has at
    // least four tiles.  The copies are added in copy order at the end.
    using acc_t = std::conditional_t<F16, floatx4, floatx16>;
    constexpr int AR = F16 ? 4 : 16;
    constexpr int NC = NF * NF >= 4 ? 1 : 4;
    acc_t acc[NC][NF][NF];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int i = 0; i < NF; ++i)
#pragma unroll
            for (int j = 0; j < NF; ++j)
#pragma unroll
                for (int r = 0; r < AR; ++r) acc[c][i][j][r] = 0.0f;

    u32x4 fa[2][NSUB][NF], fb[2][NSUB][NF];
    auto read_step = [&](int buf, int st) {
#pragma unroll
        for (int s = 0; s < NSUB; ++s)
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                fb[buf][s][f] = frag(false, st, s, f);
                fa[buf][s][f] = frag(true, st, s, f);
            }
    };
    // order: sub-step, (fp32: element e,) row tile i, column tile j
    auto mfma_sub = [&](int buf, int s) {
        if constexpr (F16) {
#pragma unroll
            for (int i = 0; i < NF; ++i)
#pragma unroll
                for (int j = 0; j < NF; ++j)
                    acc[0][i][j] = mfma_16x16x32<T>(fb[buf][s][j], fa[buf][s][i], acc[0][i][j]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < NF; ++i)
#pragma unroll
                    for (int j = 0; j < NF; ++j)
                        acc[e % NC][i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            __uint_as_float(fb[buf][s][j][e]), __uint_as_float(fa[buf][s][i][e]),
                            acc[e % NC][i][j], 0, 0, 0);
        }
    };
    auto mfma_step = [&](int buf) {
#pragma unroll
        for (int s = 0; s < NSUB; ++s) mfma_sub(buf, s);
    };
    // fp32: the MFMAs of sub-step s (mfma_sub's order) with the DMA
    // instructions [d0, d1) of step jj (into stage st; instruction d copies
    // operand A for even d, B for odd, its instruction d / 2) spread evenly
    // among them, each MFMA and its companions fenced by a sched_barrier.  A
    // step's DMA issued in one burst backs up in the texture address unit and
    // holds the wave's MFMA issue meanwhile.
    auto mfma_sub_dma = [&](int buf, int s, bool dma_on, int jj, int st, int d0, int d1) {
        if constexpr (!F16) {
            constexpr int NM = 4 * NF * NF;   // MFMAs per sub-step
            const int nd = d1 - d0;
            int k = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int i = 0; i < NF; ++i)
#pragma unroll
                    for (int jt = 0; jt < NF; ++jt) {
                        acc[e % NC][i][jt] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                            __uint_as_float(fb[buf][s][jt][e]), __uint_as_float(fa[buf][s][i][e]),
                            acc[e % NC][i][jt], 0, 0, 0);
                        if (dma_on) {
#pragma unroll
                            for (int d = 0; d < ND; ++d)
                                if (d >= d0 && d < d1 && (d - d0) * NM >= k * nd && (d - d0) * NM < (k + 1) * nd)
                                    dma_op((d & 1) == 0, jj, st, d >> 1);
                        }
                        ++k;
                        __builtin_amdgcn_sched_barrier(0);
                    }
        }
    };
    // fp32: the DMA of one step spread over the first DS sub-steps of another
    auto mfma_step_dma = [&](int buf, int ds, bool dma_on, int jj, int st) {
#pragma unroll
        for (int s = 0; s < NSUB; ++s)
            mfma_sub_dma(buf, s, dma_on, jj, st, s < ds ? (ND * s) / ds : ND, s < ds ? (ND * (s + 1)) / ds : ND);
    };

    // ---- K loop: step j in stage j % S; the DMA of step j + S - 1 goes
    // into the stage step j - 1 used (its fragments were consumed by the
    // MFMAs of step j - 1).  S >= 3: the fragments of step j + 1 are read
    // while the MFMAs of step j run. ----
#pragma unroll
    for (int j = 0; j < S - 1; ++j)
        if (j < n) dma_step(j, j);
    if constexpr (S >= 3) {
        if (n > 0) {
            wait_steps(min(S - 2, n - 1));
            read_step(0, 0);
        }
        // fragment buffer of step j: j & 1, a constant in each half of the
        // two-step loop body (a loop-carried index would put the fragment
        // arrays in scratch).  The sched_barrier keeps the MFMAs of step j,
        // and so the waits for the fragments they read, ahead of the DMA
        // that next overwrites step j's stage.
        // fp32 issues the DMA of step j + S - 1 spread over the four
        // sub-steps of step j, after the wait and the reads of step j + 1
        // (issued before it, step j + S - 2 may stay in flight: one step
        // fewer than with the burst first).  Measured (M = N = 256, K = 65536,
        // split 4, 32x32 tiles, pass 1 alone, one box): 97.4 -> 85.1 us (the
        // DMA over the first one / two sub-steps: 90.4 / 87.2); 16-bit level
        // (fp16 35.2 -> 34.6-35.0 us), so it keeps the burst.
        auto body = [&](int j, auto cur) {
            constexpr int C = decltype(cur)::value;
            if constexpr (F16) {
                if (j + S - 1 < n) dma_step(j + S - 1, (j + S - 1) % S);
                if (j + 1 < n) {
                    wait_steps(min(S - 2, n - 2 - j));
                    read_step(C ^ 1, (j + 1) % S);
                }
                mfma_step(C);
            } else {
                if (j + 1 < n) {
                    wait_steps(min(S - 3, n - 2 - j));
                    read_step(C ^ 1, (j + 1) % S);
                }
                mfma_step_dma(C, NSUB, j + S - 1 < n, j + S - 1, (j + S - 1) % S);
            }
            __builtin_amdgcn_sched_barrier(0);
        };
#pragma clang loop unroll(disable)
        for (int j = 0; j < n; j += 2) {
            body(j, std::integral_constant<int, 0>{});
            if (j + 1 < n) body(j + 1, std::integral_constant<int, 1>{});
        }
    } else {
        // two stages.  16-bit: the DMA of step j + 1 goes out at the start of
        // step j, which then waits for its own step and reads its fragments
        // (reading them one sub-step ahead instead, the first of step j + 1
        // during the last of step j: fp16 M = N = 256, split 16, 19.2 -> 22.1
        // us).  fp32: step j waits for its own DMA (issued during step j - 1),
        // reads its fragments, and spreads the DMA of step j + 1 over its
        // first two sub-steps, which leaves the last two for that DMA to land.
        // Measured (M = N = 256, K = 65536, split 16, 64x64 tiles, pass 1
        // alone, one box): 75.5-77.7 -> 68.0-70.4 us (over one sub-step 69.9-
        // 70.8, over all four 73.9); fp16 the same way 18.8-19.6 -> 22.6 us.
#pragma clang loop unroll(disable)
        for (int j = 0; j < n; ++j) {
            if constexpr (F16) {
                if (j + 1 < n) dma_step(j + 1, (j + 1) & 1);
                wait_steps(j + 1 < n ? 1 : 0);
                read_step(0, j & 1);
                mfma_step(0);
            } else {
                wait_steps(0);
                read_step(0, j & 1);
                mfma_step_dma(0, 2, j + 1 < n, j + 1, (j + 1) & 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    // ---- the four waves' sums, added in wave order ----
    // Each wave writes its TT x TT sums into its own LDS region (its DMA has
    // landed and its reads are done: no other wave uses the region), rows
    // padded by 16 bytes so the MFMA-layout writes spread over the banks.
    constexpr int RS = TT * 4 + 16;   // bytes per row
    static_assert(TT * RS <= WU * 16, "sums exceed a wave's LDS region");
    char* wl = (char*)lds + wbase * 16;
#pragma unroll
    for (int i = 0; i < NF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            acc_t a = acc[0][i][j];
#pragma unroll
            for (int c = 1; c < NC; ++c) a += acc[c][i][j];
            if constexpr (F16) {
                const int m = 16 * i + q, nn = 16 * j + 4 * g;
                *(floatx4*)(wl + m * RS + nn * 4) = a;
            } else {
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    const int m = 32 * i + l32, nn = 32 * j + 8 * qq + 4 * h;
                    *(floatx4*)(wl + m * RS + nn * 4) = floatx4{a[4 * qq], a[4 * qq + 1], a[4 * qq + 2], a[4 * qq + 3]};
                }
            }
        }
    __syncthreads();
    // wave w sums rows [w TT / 4, (w + 1) TT / 4) over the four regions
    constexpr int V4 = TT / 4;                 // float4 per row
    constexpr int PER = (TT / 4) * V4 / 64;    // float4 per lane
    float* Cp = (float*)p.C + (int64_t)b * p.s_split;
    floatx4 sum[PER];
#pragma unroll
    for (int it = 0; it < PER; ++it) {
        const int e = it * 64 + lane;
        const int r = wave * (TT / 4) + e / V4, c = e % V4;
        sum[it] = *(const floatx4*)((const char*)lds + r * RS + c * 16);
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const floatx4 v = *(const floatx4*)((const char*)lds + w * WU * 16 + r * RS + c * 16);
            sum[it] += v;
        }
    }
    if (nq == 1) {
#pragma unroll
        for (int it = 0; it < PER; ++it) {
            const int e = it * 64 + lane;
            const int r = wave * (TT / 4) + e / V4, c = e % V4;
            *(floatx4*)(Cp + (int64_t)(m0 + r) * p.ldc + n0 + 4 * c) = sum[it];
        }
        return;
    }
    // Part q of nq: store the sum (row-major TT x TT) where the other parts
    // of this slice and tile will read it, with device-scope coherent stores
    // (sc1: through the XCD's L2, which another XCD does not see), wait for
    // them, then count this workgroup's arrival.  The last of the nq to
    // arrive reads the nq sums back (device-scope coherent loads), adds them
    // in part order and writes the slice's partial: the same order whatever
    // the order of arrival, so the partials are bitwise reproducible.  The
    // counter gains nq per launch and starts each launch at a multiple of nq.
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.qpart + (int64_t)(b * per + t) * nq * (TT * TT)), (short)0, -1, 0x00020000);
    constexpr int SC1 = 16;   // cache policy: sc1 (device scope)
#pragma unroll
    for (int it = 0; it < PER; ++it) {
        const int e = it * 64 + lane;
        const int r = wave * (TT / 4) + e / V4, c = e % V4;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum[it]), rq,
                                               (int)((qi * (TT * TT) + r * TT + 4 * c) * 4), 0, SC1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __shared__ uint32_t q_last;
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(p.qcnt + b * per + t, 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        q_last = old % nq == nq - 1;
    }
    __syncthreads();
    if (!q_last) return;
#pragma unroll
    for (int it = 0; it < PER; ++it) {
        const int e = it * 64 + lane;
        const int r = wave * (TT / 4) + e / V4, c = e % V4;
        floatx4 v[WAVEK_NQ];
#pragma unroll
        for (int q = 0; q < WAVEK_NQ; ++q)
            v[q] = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(rq, (q * (TT * TT) + r * TT + 4 * c) * 4, 0, SC1));
        floatx4 tot = v[0];
#pragma unroll
        for (int q = 1; q < WAVEK_NQ; ++q) tot += v[q];
        *(floatx4*)(Cp + (int64_t)(m0 + r) * p.ldc + n0 + 4 * c) = tot;
    }
}

}  // namespace vkb
