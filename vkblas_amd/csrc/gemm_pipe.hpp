// gemm_pipe.hpp — software-pipelined 256x256 GEMM for gfx950, fp32, fp16 and
// bf16, and its 128x128 form.
//
// Used where M, N >= the tile (edge tiles move back inside the matrix and
// mask their stores), K is a multiple of two K steps and the operands are
// aligned; also as split-K pass 1 (one K slice per workgroup row of the grid,
// raw fp32 sums).  Small and unaligned shapes use gemm_kernel<> in
// gemm_mfma.hpp, whose MFMA role swap and epilogue this kernel shares.
// Replaces the reference's large tiles (gemm_f32_128x128_bankfree_tmpl.comp,
// gemm_half_128x256_bankfree_tmpl.comp, gemm_half_128x128_bankfree_tmpl.comp,
// dispatched from src/vkblas.c:1191-1313, 1822-1868).
//
// Per workgroup: 4 waves, 2x2, each owning a WT x WT block of C (WT = 128:
// 256 AGPRs; WT = 64: 64 AGPRs, two workgroups per CU).  A K step is 128
// bytes of K (64 fp16 / bf16 or 32 fp32):
//  * 16-bit types, every layout: two sub-steps of v_mfma_f32_16x16x32 on 8x8
//    (WT 64: 4x4) 16x16 tiles (lane group g = lane / 16 takes k 8g..8g+7 of
//    the sub-step's 32);
//  * fp32: four sub-steps of v_mfma_f32_32x32x2_f32 on 4x4 (WT 64: 2x2)
//    32x32 tiles; MFMA e of sub-step s takes k = 8 s + e from lanes 0-31 and
//    k = 8 s + 4 + e from lanes 32-63.
// Per K step:
//  * Operand tiles go global -> LDS directly (buffer_load ... lds: lane l of
//    a wave writes 16 B at M0 + 16 l), so they use no VGPRs and no ds_write;
//    lane l fetches the global chunk that the LDS swizzle maps to its slot,
//    so the global side stays fully coalesced.
//  * An fp32 MN-major operand stays MN-major in LDS: the 32x32x2 MFMA takes
//    one element per lane and k, and 32 lanes of one k row read 32
//    consecutive m, so its fragments are ds_read_b32 of whole 128-byte row
//    segments.
//  * A 16-bit MN-major operand stays MN-major in LDS and its fragments are
//    read with ds_read_b64_tr_b16: within each 16-lane group, lane i receives
//    element i & 3 of the 8 bytes addressed by lanes (i >> 2) + 4 j, j = 0..3.
//    Lane q of group g addressing row k = 8g + (q >> 2) (+4 for the second
//    read), columns 4 (q & 3) .. +3 of the fragment, therefore receives k
//    8g .. 8g+3 (then +4 .. +7) of column q: the MFMA operand layout.
//  * Loads for K step t+1 are issued during step t into the other LDS stage;
//    MFMA fragments for sub-step s+1 are read from LDS while the MFMAs of
//    sub-step s run (two register sets).
//  * One barrier per K step.
//
// LDS map (16-byte units): A stage s at s*2304, B stage s at 4608 + s*2304
// (144 KB).  gfx950's LDS is 64 banks (256 bytes) wide and serves a
// ds_read_b128 16 lanes at a time, so the 16 rows a fragment read touches at
// one chunk must land on 16 distinct 16-byte bank groups: the 8 rows of one
// row parity share a 256-byte bank line half and need 8 distinct slots.
//  * fp32 MN-major tiles (k rows of BM m, unswizzled): BM 256: row k at
//    k * 1056 bytes (one DMA instruction per row); BM 128: rows k, k+1 form
//    a 1-KiB block (one instruction) at (k >> 1) * 1088, row k & 1 at +512.
//    A fragment read has lanes 0-31 on row k and lanes 32-63 on row k + 4:
//    4 * 1056 and 2 * 1088 are 128 modulo 256, so the two 128-byte segments
//    fall on the two halves of the 64 banks.
//  * K-major tiles (written by whole-row DMA, lane l -> +16 l, so the swizzle
//    can only depend on r & 7): chunk c of row r at slot c ^ (r & 7), rows
//    in groups of 8 at (r >> 3)*GRP + (r & 7)*8.  16-bit types read 16-row
//    fragments and use GRP = 64 (no padding): measured free of bank
//    conflicts, while a 128-byte pad per group gives them 1.5x the LDS read
//    time.  fp32 reads 32-row fragments and uses GRP = 72 (1152-byte group
//    stride): the pad moves odd groups to the other half of the bank line,
//    which separates rows r and r + 8 that share r & 7.
//  * 16-bit MN-major tiles (k rows of 256 m or n, 32 chunks): rows k, k+1
//    form a 1-KiB block (one DMA instruction) at (k >> 1)*64, row k & 1 at
//    +32, chunk c at slot c ^ t(k), t(k) = 2 (k & 3) + 8 (((k >> 3) ^
//    (k >> 4)) & 1).  A transposing read of 32 lanes touches rows
//    {8g + 0..3} of two lane groups at two chunks 2i, 2i + 1: t takes 8
//    distinct even values over those rows for either pairing of the four
//    groups ((0,1)(2,3) or (0,2)(1,3)), so the 16 chunks fall on 16 distinct
//    16-byte bank groups.  t(k + 4) = t(k) for the second read and
//    t(k + 32) = t(k) for the second sub-step, so both are immediate offsets.
// Every row base has its low three bits clear, so a fragment's slot index is
// (base + (hoff ^ g)) ^ sub-step offset (4s for 16-bit types, 2s for fp32).
//
// Global traffic uses buffer loads on resources based at the tile's first
// element: a fixed per-lane VGPR offset plus a uniform SGPR offset (row step
// and k0), so the loop does no 64-bit address arithmetic.
#pragma once
#include <type_traits>
#include "gemm_mfma.hpp"

namespace vkb {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Lane id within the wave, computed by instructions the compiler cannot
// merge with an earlier computation (a fresh value where keeping the old one
// live would cost registers).
__device__ __forceinline__ int fresh_lane_id() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;
typedef __attribute__((address_space(3))) const uint32_t lds_u32_t;

#ifndef VKB_PIPE_DMA_UNITS
#define VKB_PIPE_DMA_UNITS 16
#endif

// Read order of the SH 0 fragments of a sub-step: units in order, each
// needing B_j (its MFMAs' columns) then A_i (its row) on first use.
struct RdSeq {
    int n;
    signed char isA[16], fi[16];
};
template <int NF>
constexpr RdSeq make_rdseq() {
    RdSeq r{};
    bool seenA[8] = {}, seenB[8] = {};
    constexpr int MPU = NF * NF / 16;   // MFMAs per unit
    for (int q = 0; q < 16; ++q) {
        const int t0 = q * MPU, i = t0 / NF, j0 = t0 % NF;
        for (int j = j0; j < j0 + MPU; ++j)
            if (!seenB[j]) { seenB[j] = true; r.isA[r.n] = 0; r.fi[r.n] = (signed char)j; ++r.n; }
        if (!seenA[i]) { seenA[i] = true; r.isA[r.n] = 1; r.fi[r.n] = (signed char)i; ++r.n; }
    }
    return r;
}

// WT: wave tile edge.  128: 256x256 workgroup tile, one workgroup per CU;
// 64: 128x128 workgroup tile for shapes with too few 256x256 tiles to fill
// the chip (fp32 always with two stages).
// NST: LDS stages.  2: the DMA of a K step is issued one step ahead.  4
// (WT 64 only, 144 KB: one workgroup per CU, for grids of at most one
// workgroup per CU): three steps ahead, since a 128x128 step (512 MFMA
// cycles) is shorter than the load latency.
template <typename T, typename TC, bool AK, bool BKM, int WT = 128, int NST = 2>
__global__ __launch_bounds__(256, (WT == 128 || NST == 4) ? 1 : 2) void gemm_pipe_kernel(KParams p) {
    constexpr bool F16 = sizeof(T) == 2;
    static_assert(WT == 128 || WT == 64, "256x256 or 128x128 tiles");
    static_assert(NST == 2 || (NST == 4 && WT == 64 && F16), "four stages: 16-bit 128x128 tiles only");
    constexpr int ES = sizeof(T);                   // element bytes
    constexpr int BM = 2 * WT, BN = 2 * WT, BK = 128 / ES;
    constexpr int NDMA = BM / 32;                   // DMA instructions per operand, wave and K step
    constexpr int CPR = BM / 8;                     // 16-byte chunks of an MN-major k row
    constexpr int RPB = 64 / CPR;                   // k rows per 1-KiB transposed-read block
    constexpr int STG = (BM / 8) * 72;              // stage size (u32x4), every layout fits
    constexpr int A0 = 0, B0 = NST * STG;           // u32x4 offsets: A stages, then B stages
    constexpr int GRP = F16 ? 64 : 72;              // 8-row group stride of K-major tiles
    __shared__ u32x4 lds[2 * NST * STG];            // 144 KB (BM 256; BM 128 x 4 stages) / 72 KB

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
    const uint32_t b = bid / per;                   // batch, or K slice under split-K
    const uint32_t t = bid - b * per;
    // tiles are walked in groups of GM tile-rows; 4 measured 0-2% faster than
    // 8 at 4096^3 and 8192^3 (2 and 16 slower)
    constexpr uint32_t GM = 4;
    const uint32_t width = GM * p.tiles_n;
    const uint32_t group = t / width;
    const uint32_t first_m = group * GM;
    const uint32_t gm = min(p.tiles_m - first_m, GM);
    const uint32_t tin = t - group * width;
    // Edge tiles (M or N not a multiple of the tile, M >= BM and N >= BN:
    // the launcher checks) move back inside the matrix, so every load stays
    // in bounds: the last tile row computes rows M - BM .. M - 1 and stores
    // only those from its own start m_lo on, which the tile before it does
    // not store (likewise for columns).  Nothing is stored twice, so beta
    // != 0 reads each C element once.
    // Short M (128x128 tiles with K-major A only, M < BM): the one tile row
    // starts at row 0, A rows past M - 1 are read as row M - 1 and C rows
    // from M on are not stored.
    const int m_lo = (int)(first_m + tin % gm) * BM;
    const int n_lo = (int)(tin / gm) * BN;
    const int m0 = max(0, min(m_lo, (int)p.M - BM));
    const int n0 = min(n_lo, (int)p.N - BN);

    const int lda = (int)p.lda, ldb = (int)p.ldb;
    // Split-K pass 1 (split > 1, batch 1): slice b covers k in
    // [b kps, min(K, (b + 1) kps)) and writes raw sums to C + b s_split.  The
    // launcher makes kps and K multiples of two K steps, so every slice is.
    const bool sk = p.split > 1;
    const int64_t kbeg = sk ? (int64_t)b * p.kps : 0;
    const uint32_t klen = sk ? min(p.K - (uint32_t)kbeg, p.kps) : p.K;
    const int64_t bat = sk ? 0 : (int64_t)b;
    // Buffer resources on the tile's first element; all per-lane parts are
    // 32-bit byte offsets (the launcher guarantees they fit).
    const T* At = (const T*)p.A + bat * p.sa + (AK ? (int64_t)m0 * p.lda + kbeg : kbeg * p.lda + m0);
    const T* Bt = (const T*)p.B + bat * p.sb + (BKM ? (int64_t)n0 * p.ldb + kbeg : kbeg * p.ldb + n0);
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc((void*)At, (short)0, -1, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc((void*)Bt, (short)0, -1, 0x00020000);
    TC* Cb = (TC*)p.C + (sk ? (int64_t)b * p.s_split : (int64_t)b * p.sc);
    const int nkt = (int)(klen / BK);

    // K-major direct loads: instruction i of this wave fills the 8-row group
    // NDMA wave + i (rows (BM / 4) wave + 8 i + [0, 8); lane -> row + lane / 8,
    // slot lane % 8).  With the K-major swizzle c ^ (r & 7) that slot holds
    // chunk (lane % 8) ^ (lane / 8) for every i, so one VGPR offset serves
    // every instruction; the row step 8 i and k0 go in soffset.
    const int koff = ((lane & 7) ^ (lane >> 3)) << 4;
    const int a_voff = ((BM / 4) * wave + (lane >> 3)) * lda * ES + koff;
    // 128x128 tiles: one VGPR offset per instruction, its row clamped to the
    // last row of A (a no-op unless M < BM)
    constexpr int NAV = (WT == 64 && AK) ? NDMA : 1;
    int a_vn[NAV];
#pragma unroll
    for (int n = 0; n < NAV; ++n)
        a_vn[n] = min((BM / 4) * wave + (lane >> 3) + 8 * n, (int)p.M - 1 - m0) * lda * ES + koff;
    const int b_voff = ((BN / 4) * wave + (lane >> 3)) * ldb * ES + koff;
    // 16-bit MN-major direct loads: instruction n of this wave fills the
    // 1-KiB block NDMA wave + n (k rows RPB (NDMA wave + n) + [0, RPB); lane ->
    // row + lane / CPR, slot lane % CPR, which holds chunk
    // (lane % CPR) ^ t(row)).  t(row) depends on n only through n & 1 and
    // n >> 2 (BM 256) or n >> 1 (BM 128), so four or two VGPR offsets serve
    // the instructions; the row step and k0 go in soffset.
    constexpr bool ATR = F16 && !AK, BTR = F16 && !BKM;
    auto tsw = [](int k) { return 2 * (k & 3) + 8 * (((k >> 3) ^ (k >> 4)) & 1); };
    constexpr int NTRV = WT == 128 ? 4 : 2;
    auto trv = [](int n) { return WT == 128 ? ((n & 1) | ((n >> 2) << 1)) : ((n >> 1) & 1); };
    int a_tr[NTRV], b_tr[NTRV];
#pragma unroll
    for (int v = 0; v < NTRV; ++v) {
        const int n = WT == 128 ? ((v & 1) | ((v >> 1) << 2)) : 2 * v;   // an instruction of variant v
        const int r = lane / CPR;
        const int k = RPB * (NDMA * wave + n) + r;
        a_tr[v] = r * lda * ES + (((lane % CPR) ^ tsw(k)) << 4);
        b_tr[v] = r * ldb * ES + (((lane % CPR) ^ tsw(k)) << 4);
    }
    // fp32 MN-major direct loads: instruction n of this wave fills k row
    // NDMA wave + n (BM 256: lane -> m chunk lane) or the two-row block
    // NDMA wave + n (BM 128: lane -> row lane / 32, m chunk lane % 32); one
    // VGPR offset serves every instruction, the row and k0 go in soffset.
    constexpr bool AMN = !F16 && !AK, BMN = !F16 && !BKM;
    constexpr int MNB = BM == 256 ? 66 : 68;        // u32x4 units per row (BM 256) or row pair (BM 128)
    constexpr int MNR = BM == 256 ? 1 : 2;          // k rows per DMA instruction
    auto mn_unit = [](int k) { return BM == 256 ? k * 66 : (k >> 1) * 68 + (k & 1) * 32; };
    const int a_mnoff = BM == 256 ? lane * 16 : (lane >> 5) * lda * ES + (lane & 31) * 16;
    const int b_mnoff = BM == 256 ? lane * 16 : (lane >> 5) * ldb * ES + (lane & 31) * 16;

    // Barrier after "s_waitcnt vmcnt(n) lgkmcnt(0)": n counts the DMA of
    // later K steps that may stay in flight; vector loads complete in issue
    // order, so this still waits for the step's own DMA.  The barrier is
    // written out (no __syncthreads) because its workgroup fence would wait
    // for every outstanding load; the "memory" clobber keeps the compiler
    // from moving LDS accesses across it.
    auto sync_vm = [](auto n_c) {
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(decltype(n_c)::value) : "memory");
    };

    // With a transposed-read operand or more than two stages every DMA is
    // issued as inline assembly.  The compiler waits for all LDS DMA in
    // flight (vmcnt) before each ds_read_b64_tr_b16 it emits, which would
    // serialize the loads behind the reads, and it cannot tell which stage a
    // DMA writes; as assembly the DMA is outside its wait-count tracking.
    // The end-of-step "s_waitcnt vmcnt(n)" + barrier (sync_vm) is what orders
    // a step's DMA before any read of its stage (n counts the DMA of later
    // steps, issued after it: vector loads complete in order), and these
    // kernels have no other vector-memory load in flight in the K loop.
    constexpr bool ASM_DMA = ATR || BTR || NST > 2;
    auto rsrc_words = [](const void* base) {
        const uint64_t a = (uint64_t)base;
        return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                     __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32) & 0xffff), -1, 0x00020000};
    };
    const i32x4 ra_w = rsrc_words(At), rb_w = rsrc_words(Bt);
    auto dma = [&](bool isA, lds_ptr_t dst, int voff, int soff) {
        if constexpr (ASM_DMA) {
            const int m0 = __builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)dst);
            asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
                         :: "v"(voff), "s"(isA ? ra_w : rb_w), "s"(__builtin_amdgcn_readfirstlane(soff)),
                            "{m0}"(m0));
        } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(isA ? ra : rb, dst, 16, voff, soff, 0, 0);
        }
    };
    // Direct (DMA) load n of K step kt (NDMA per operand per wave: A then B)
    constexpr int ND = 2 * NDMA;
    auto dma_load = [&](int kt, int S, int n) {
        const int k0 = kt * BK;
        if (n < NDMA) {
            if constexpr (AK && NAV > 1)
                dma(true, (lds_ptr_t)&lds[A0 + S * STG + (NDMA * wave + n) * GRP], a_vn[n], k0 * ES);
            else if constexpr (AK)
                dma(true, (lds_ptr_t)&lds[A0 + S * STG + (NDMA * wave + n) * GRP], a_voff, (k0 + n * 8 * lda) * ES);
            else if constexpr (ATR)
                dma(true, (lds_ptr_t)&lds[A0 + S * STG + (NDMA * wave + n) * 64], a_tr[trv(n)],
                    (k0 + RPB * (NDMA * wave + n)) * lda * ES);
            else
                dma(true, (lds_ptr_t)&lds[A0 + S * STG + (NDMA * wave + n) * MNB], a_mnoff,
                    (k0 + MNR * (NDMA * wave + n)) * lda * ES);
        } else {
            const int m = n - NDMA;
            if constexpr (BKM)
                dma(false, (lds_ptr_t)&lds[B0 + S * STG + (NDMA * wave + m) * GRP], b_voff, (k0 + m * 8 * ldb) * ES);
            else if constexpr (BTR)
                dma(false, (lds_ptr_t)&lds[B0 + S * STG + (NDMA * wave + m) * 64], b_tr[trv(m)],
                    (k0 + RPB * (NDMA * wave + m)) * ldb * ES);
            else
                dma(false, (lds_ptr_t)&lds[B0 + S * STG + (NDMA * wave + m) * MNB], b_mnoff,
                    (k0 + MNR * (NDMA * wave + m)) * ldb * ES);
        }
    };

    // ---- MFMA shape --------------------------------------------------------
    // SH 0, 16-bit types: v_mfma_f32_16x16x32; a sub-step is one 32-wide k
    //   slice (lane group g = lane / 16 holds 8 k of row lane % 16); the
    //   wave's WT x WT block is NF x NF tiles of 16x16 (floatx4).  With random
    //   data gfx950 sustains ~15% more fp16 FLOP/s on 16x16x32 than on
    //   32x32x16 (half the accumulator traffic per FLOP under the power limit).
    // SH 2, fp32: v_mfma_f32_32x32x2_f32, NF x NF tiles of 32x32 (4x4 for WT
    //   128, 2x2 for WT 64).  In sub-step s lane half h holds k 8s + 4h .. +3
    //   of its row (a K-major fragment is chunk 2s + h) and MFMA e takes
    //   element e.
    constexpr int SH = F16 ? 0 : 2;
    constexpr int NSUB = SH == 0 ? 2 : 4;           // sub-steps per K step
    constexpr int UPS = 32 / NSUB;                  // units per sub-step
    constexpr int NF = WT / (SH == 0 ? 16 : 32);    // fragments per operand
    constexpr int MPU = NF * NF / 16;               // MFMAs per unit (SH 0)
    constexpr int FR = SH == 0 ? 16 : 32;           // rows per fragment
    constexpr int SX = SH == 0 ? 4 : 2;             // sub-step slot offset
    const int fl = SH == 0 ? (lane & 15) : l32;     // fragment row of this lane
    const int hoff = SH == 0 ? (lane >> 4) : h;     // chunk in sub-step 0

    // K-major fragment slot of row r: row base + (hoff ^ (r & 7)); sub-step s
    // reads it ^ (s * SX).  Fragment i starts FR rows further on (FR = 16 or
    // 32, a multiple of 8), which moves the row base by the constant STEP and
    // leaves r & 7 alone, so STEP i goes in the ds_read immediate offset.
    auto row_base = [&](int r) { return (r >> 3) * GRP + (r & 7) * 8; };
    constexpr int STEP = (FR / 8) * GRP;
    int xa[8], xb[8];   // indexed by the slot XOR; unused entries are dead code
    {
        const int ra = wm * WT + fl, rb = wn * WT + fl;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            xa[c] = A0 + row_base(ra) + ((hoff ^ (ra & 7)) ^ c);
            xb[c] = B0 + row_base(rb) + ((hoff ^ (rb & 7)) ^ c);
        }
    }
    // fp32 MN-major fragments: lane (l32, h) reads m = (wave's m) + 32 i + l32
    // of k row 8 s + 4 h + e for MFMA e: a per-lane byte base with row 4 h;
    // the k row 8 s + e, fragment i (+128 bytes) and the stage are offsets.
    const int a_mnb = mn_unit(4 * h) * 16 + (wm * WT + l32) * 4;
    const int b_mnb = mn_unit(4 * h) * 16 + (wn * WT + l32) * 4;
    // Transposed-read fragments (16-bit MN-major tiles): lane q of group g
    // reads row k = 8g + (q >> 2) at columns 16 i + 4 (q & 3) .. +3 of the
    // wave's WT; its unit is (k / RPB) 64 + (k % RPB) CPR + (c ^ t(k)) with
    // c = (WT / 8) w + 2 i + ((q >> 1) & 1) and t(k) = 2 (q >> 2) +
    // 8 ((g ^ g >> 1) & 1) (even, below 16), plus 8 bytes for odd q.  Per
    // fragment i that is a per-lane base with ((WT / 8) w + 2 i) ^ t; the
    // second read (+4 rows), the second sub-step (+32 rows) and the stage are
    // offsets (TR_HALF, TR_SUB bytes).
    constexpr int TR_HALF = (4 / RPB) * 64 * 16, TR_SUB = (32 / RPB) * 64 * 16;
    int tra[NF], trb[NF];   // bytes
    {
        const int g = lane >> 4, q = lane & 15;
        const int tk = 2 * (q >> 2) + 8 * ((g ^ (g >> 1)) & 1);
        const int k = 8 * g + (q >> 2);
        const int L = (k / RPB) * 64 + (k % RPB) * CPR + ((q >> 1) & 1);
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            tra[i] = (A0 + L + (((WT / 8) * wm + 2 * i) ^ tk)) * 16 + (q & 1) * 8;
            trb[i] = (B0 + L + (((WT / 8) * wn + 2 * i) ^ tk)) * 16 + (q & 1) * 8;
        }
    }

    using acc_t = std::conditional_t<SH == 0, floatx4, floatx16>;
    constexpr int AR = SH == 0 ? 4 : 16;            // accumulator registers per tile
    acc_t acc[NF][NF];
#pragma unroll
    for (int i = 0; i < NF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j)
#pragma unroll
            for (int r = 0; r < AR; ++r) acc[i][j][r] = 0.0f;

    // A sub-step is UPS units; its units also read the fragments of the next
    // sub-step, in the order the next sub-step first uses them.
    // SH 0: unit q = MPU tiles from tile q MPU (row-major over NF x NF): with
    //   WT 128 tiles (q/2, 4(q%2) .. +3), reads B0-B3 A0 B4-B7 A1 .. A7; with
    //   WT 64 tile (q/4, q%4), reads B0 A0 B1 B2 B3 A1 A2 A3.  A
    //   transposed-read fragment is two reads; the NRD reads are dealt over
    //   the 16 units in order.  With WT 128 and K-major A, A_i is last used by
    //   unit 2i+1 and its successor is read in that unit or a later one, so A
    //   needs one register set; otherwise A is read earlier and takes two, as
    //   B always does.
    // SH 2: unit q = k element q/2 of the chunk on tile rows (NF/2)(q%2) ..
    //   +NF/2 - 1, all NF columns: units 0 .. 2 NF - 1 read B0 .. B(NF-1), then
    //   A0 .. A(NF-1), every fragment kept to the sub-step's end: two sets
    //   each.
    constexpr int NAB = (SH == 0 && !ATR && WT == 128) ? 1 : 2;
    constexpr int NRD = 2 * NF + (ATR ? NF : 0) + (BTR ? NF : 0);   // SH 0 reads per sub-step
    u32x4 af[NAB][NF], bf[2][NF];
    auto tr_half = [&](u32x4& dst, int half, int byte_off) {
        const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)((char*)lds + byte_off));
        const u32x2 w = __builtin_bit_cast(u32x2, v);
        dst[2 * half] = w[0];
        dst[2 * half + 1] = w[1];
    };
    auto mn_frag = [&](u32x4& dst, int byte_off, int s) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            dst[e] = *(lds_u32_t*)((char*)lds + byte_off + mn_unit(8 * s + e) * 16);
    };
    auto frag_read = [&](int buf, int S, int s, bool isA, int fi, int half) {
        if (isA) {
            if constexpr (ATR) tr_half(af[buf % NAB][fi], half, tra[fi] + S * STG * 16 + s * TR_SUB + half * TR_HALF);
            else if constexpr (AMN) mn_frag(af[buf % NAB][fi], (A0 + S * STG) * 16 + a_mnb + 128 * fi, s);
            else af[buf % NAB][fi] = lds[xa[SX * s] + S * STG + fi * STEP];
        } else {
            if constexpr (BTR) tr_half(bf[buf][fi], half, trb[fi] + S * STG * 16 + s * TR_SUB + half * TR_HALF);
            else if constexpr (BMN) mn_frag(bf[buf][fi], (B0 + S * STG) * 16 + b_mnb + 128 * fi, s);
            else bf[buf][fi] = lds[xb[SX * s] + S * STG + fi * STEP];
        }
    };
    auto read_one = [&](int buf, int S, int s, int q) {   // the reads of unit q
        if constexpr (SH == 0) {
            constexpr RdSeq SEQ = make_rdseq<NF>();
            int o = 0;   // read index in the sub-step's sequence
#pragma unroll
            for (int t = 0; t < SEQ.n; ++t) {
                const bool tr = SEQ.isA[t] ? ATR : BTR;
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    if (half == 1 && !tr) continue;
                    if (o * 16 >= q * NRD && o * 16 < (q + 1) * NRD) frag_read(buf, S, s, SEQ.isA[t], SEQ.fi[t], half);
                    ++o;
                }
            }
        } else {
            if (q < 2 * NF) frag_read(buf, S, s, q >= NF, q % NF, 0);
        }
    };
    auto mfma_unit = [&](int buf, int q) {
        if constexpr (SH == 0) {
            const int i = (q * MPU) / NF, j0 = (q * MPU) % NF;
#pragma unroll
            for (int j = j0; j < j0 + MPU; ++j)
                acc[i][j] = mfma_16x16x32<T>(bf[buf][j], af[buf % NAB][i], acc[i][j]);
        } else {
            const int e = q >> 1, i0 = (q & 1) * (NF / 2);
#pragma unroll
            for (int i = i0; i < i0 + NF / 2; ++i)
#pragma unroll
                for (int j = 0; j < NF; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(bf[buf][j][e]),
                                                                    __uint_as_float(af[buf % NAB][i][e]), acc[i][j],
                                                                    0, 0, 0);
        }
    };

    // A region (between two barriers) is 32 units: the last sub-step of K step
    // kt-1 (units [0, UPS), from registers) and the first NSUB-1 sub-steps of
    // kt.  The ND DMA loads of kt+1 are spread over DMA_UNITS units from the
    // first (issued in a burst they oversubscribe the texture address unit
    // and stall the MFMA issue).  The first region has no previous sub-step:
    // its units start at UPS and its DMA is spread over [UPS, 24).
    // 16-bit 256x256 tiles with K-major A and transposed-read B: 24 units
    // (fp16 4096^3 -4%, 8192^3 -1%; the same spread costs the K-major /
    // K-major form 2-3% at 8192^3, and 20 units change neither).
    constexpr int DMA_UNITS = (F16 && WT == 128 && AK && !BKM) ? 24 : VKB_PIPE_DMA_UNITS;
    static_assert(DMA_UNITS >= 1 && DMA_UNITS <= 24, "DMA spread over 1 .. 24 units");
    auto dma_unit = [&](int kt, int S, int u, bool prev) {   // u: unit of the region
        const int first = prev ? 0 : UPS;
        const int span = prev ? DMA_UNITS : 24 - UPS;
        const int v = u - first;
#pragma unroll
        for (int n = 0; n < ND; ++n)
            if (n * span >= v * ND && n * span < (v + 1) * ND) dma_load(kt, S, n);
    };

    // Region, stage S = K step kt:
    //   sub-step NSUB-1 of K step kt-1 (its buffer)  + reads of (kt, 0)
    //   sub-steps 0 .. NSUB-2 of kt                  + reads of the next one
    //   DMA of kt+1 -> stage S^1
    //   wait for this wave's DMA and LDS traffic, barrier
    // Sub-step s of K step kt uses fragment buffer s & 1 (NSUB is even).
    // Every unit (MFMAs + companions) is fenced with sched_barrier so the
    // compiler keeps this order and both fragment sets live.
    // next: this region issues the DMA of step kt + NST - 1 (into the stage
    // step kt - 1 used); wc: the vmcnt that leaves step kt + 1 landed.
    auto region = [&](int kt, int S, bool prev, bool next, auto wc) {
#pragma unroll
        for (int u = prev ? 0 : UPS; u < 32; ++u) {
            const int sub = u / UPS - 1;          // sub-step of kt run here (-1: kt-1's last)
            const int q = u % UPS;
            const int buf = sub < 0 ? (NSUB - 1) & 1 : sub & 1;
            mfma_unit(buf, q);
            read_one((sub + 1) & 1, S, sub + 1, q);
            // the step is clamped for the 16-bit two-stage loop, whose last
            // region re-reads step nkt - 1 into the idle stage (below)
            if (next) dma_unit(min(kt + NST - 1, nkt - 1), (S + NST - 1) % NST, u, prev);
            __builtin_amdgcn_sched_barrier(0);
        }
        sync_vm(wc);
    };
    using W0 = std::integral_constant<int, 0>;

    // ---- prologue: K step 0 into stage 0 (NST 4: steps 1 and 2 too) ----
#pragma unroll
    for (int n = 0; n < ND; ++n) dma_load(0, 0, n);
    if constexpr (NST == 4) {
        // steps 1 and 2 as well (nkt >= 4), or step 1 only (nkt == 2)
#pragma unroll
        for (int n = 0; n < ND; ++n) dma_load(1, 1, n);
        if (nkt > 2) {
#pragma unroll
            for (int n = 0; n < ND; ++n) dma_load(2, 2, n);
            sync_vm(std::integral_constant<int, 2 * ND>{});
        } else {
            sync_vm(std::integral_constant<int, ND>{});
        }
    } else {
        sync_vm(W0{});
    }
#pragma unroll
    for (int q = 0; q < UPS; ++q) read_one(0, 0, 0, q);

    // nkt is even: regions cycle through the stages; the loop body is
    // branch-free, the last regions load less
    if constexpr (NST == 4) {
        using W1 = std::integral_constant<int, ND>;
        using W2 = std::integral_constant<int, 2 * ND>;
        if (nkt == 2) {
            region(0, 0, false, false, W0{});
            region(1, 1, true, false, W0{});
        } else {
            region(0, 0, false, true, W2{});   // loads step 3
            int kt = 1;
#pragma clang loop unroll(disable)
            for (; kt + 3 < nkt; ++kt) region(kt, kt & 3, true, true, W2{});
            region(kt, kt & 3, true, false, W1{});             // kt == nkt - 3
            region(kt + 1, (kt + 1) & 3, true, false, W0{});
            region(kt + 2, (kt + 2) & 3, true, false, W0{});
        }
    } else if (nkt == 2) {
        region(0, 0, false, true, W0{});
        region(1, 1, true, false, W0{});
    } else {
        region(0, 0, false, true, W0{});
        int kt = 1;
        if constexpr (SH == 0) {
            // One region per iteration, stage from the loop counter: with two
            // (stages 1 and 0 as constants) the register allocator gives the
            // accumulator tiles different registers in the two halves and
            // copies them around on every iteration (AGPR moves and parking
            // in VGPRs, ~100 extra VALU per two K steps).  The fp32 shape
            // keeps the constant stages (its LDS addresses fold into
            // immediates) and shows no such copies.
            // The last two regions run in the loop too: as separate code the
            // allocator gave them their own accumulator registers, with AGPR
            // moves and 1-10 spilled VGPRs (scratch writes on every call).
            // The last region's copy re-reads step nkt - 1 (from L2) into the
            // stage no later read uses; its end-of-region wait retires that
            // copy before the epilogue reuses the LDS.
#pragma clang loop unroll(disable)
            for (; kt < nkt; ++kt) region(kt, kt & 1, true, true, W0{});
        } else {
            for (; kt + 3 < nkt; kt += 2) {
                region(kt, 1, true, true, W0{});
                region(kt + 1, 0, true, true, W0{});
            }
            region(kt, 1, true, true, W0{});       // kt == nkt - 3
            region(kt + 1, 0, true, true, W0{});   // loads step nkt-1
            region(kt + 2, 1, true, false, W0{});
        }
    }
#pragma unroll
    for (int q = 0; q < UPS; ++q) mfma_unit((NSUB - 1) & 1, q);   // last sub-step of the last K step

    // ---- epilogue: C = alpha * acc (+ beta * C) ----
    // 16x16 tiles: lane holds n = 4 (lane / 16) + e of row m = lane % 16;
    // 32x32 tiles: register 4 q + e holds n = 8 q + 4 h + e of row m = l32.
    // The lane-derived indices are recomputed here from v_mbcnt (volatile
    // asm, so not merged with the prologue's): kept live across the K loop
    // instead, two of them were spilled to scratch on every call.
    {
    const int lane = fresh_lane_id();
    const int h = lane >> 5;
    const int fl = SH == 0 ? (lane & 15) : (lane & 31);
    float alpha, beta;
    load_scalars(p, alpha, beta);
    constexpr int NQ = SH == 0 ? 1 : 4;
    const float beta_u = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, beta)));
    // bias of this lane's output columns, loaded once (inside the unrolled
    // store loops the per-element loads make them too large to unroll)
    const bool has_bias = p.epi.bias != nullptr;
    float bcol[NF][NQ][4];
#pragma unroll
    for (int j = 0; j < NF; ++j)
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) bcol[j][q][e] = 0.0f;
    if (has_bias) {
        const int nb = n0 + wn * WT + (SH == 0 ? 4 * (lane >> 4) : h * 4);
#pragma unroll
        for (int j = 0; j < NF; ++j)
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int e = 0; e < 4; ++e) bcol[j][q][e] = bias_at(p.epi, nb + j * FR + q * 8 + e);
    }
    if (beta_u == 0.0f && p.c_rows16) {
        // Staged through LDS so C leaves as whole rows: the MFMA layout
        // spreads a store instruction over 16-32 rows of C, the texture
        // address unit then handles a line per row.  The rows are stored
        // non-temporal: C is not read again here, and keeping it out of L2
        // leaves room for the A and B panels other tiles still read (8192^3
        // bf16 +6%, fp16 +2-3%, 4096^3 +1-2%).  Each wave owns an LDS
        // region (the K loop's last barrier has retired every tile read) with
        // rows padded by 16 bytes: the MFMA-layout writes then fall on
        // distinct banks.  fp32 with WT 128 (512-byte rows) goes in two
        // passes of 64 rows.
        constexpr int ROWB = WT * (int)sizeof(TC);           // bytes of a wave-block row
        constexpr int STR = ROWB + 16;                       // padded LDS row stride
        constexpr int PASSES = (sizeof(TC) == 4 && WT == 128) ? 2 : 1;
        constexpr int PROWS = WT / PASSES;                   // rows per pass
        constexpr int LPR = ROWB / 16;                       // lanes per row on read-out
        static_assert(4 * PROWS * STR <= 2 * NST * STG * 16, "epilogue staging exceeds LDS");
        char* wl = (char*)lds + wave * (PROWS * STR);
        TC* cblk = Cb + (int64_t)(m0 + wm * WT) * p.ldc + (n0 + wn * WT);
#pragma unroll
        for (int pass = 0; pass < PASSES; ++pass) {
#pragma unroll
            for (int i = 0; i < NF; ++i) {
                const int m = i * FR + fl - pass * PROWS;   // row within this pass
                if (i * FR < pass * PROWS || i * FR >= (pass + 1) * PROWS) continue;
#pragma unroll
                for (int j = 0; j < NF; ++j) {
#pragma unroll
                    for (int q = 0; q < NQ; ++q) {
                        const int n = j * FR + (SH == 0 ? 4 * (lane >> 4) : q * 8 + h * 4);
                        float x[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) x[e] = alpha * acc[i][j][q * 4 + e];
                        if (has_bias) {
#pragma unroll
                            for (int e = 0; e < 4; ++e) x[e] += bcol[j][q][e];
                        }
                        store4<TC>((TC*)(wl + m * STR + n * (int)sizeof(TC)), x, true);
                    }
                }
            }
            // a wave's LDS operations complete in order; the wait keeps the
            // compiler from reordering the cross-lane read-back
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int it = 0; it < PROWS * LPR / 64; ++it) {
                const int r = it * (64 / LPR) + lane / LPR, c = lane % LPR;
                const u32x4 v = *(const u32x4*)(wl + r * STR + c * 16);
                // an edge tile's chunks start on n_lo: the launcher takes this
                // path only where N is a multiple of 16 bytes of C
                const int row = m0 + wm * WT + pass * PROWS + r;
                const bool mine = row >= m_lo && row < (int)p.M &&
                                  n0 + wn * WT + c * (16 / (int)sizeof(TC)) >= n_lo;
                if (mine)
                    __builtin_nontemporal_store(v, (u32x4*)((char*)(cblk + (int64_t)(pass * PROWS + r) * p.ldc) + c * 16));
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
    } else {
        // Direct stores of 4 consecutive n per lane (16 B fp32, 8 B 16-bit:
        // the launcher's vec_c alignment); C is read only when beta != 0, so
        // a NaN in C never reaches a beta == 0 result.  Rows that are not
        // 16-byte aligned (16-bit C with ldc % 8 == 4, or C at an 8-byte
        // offset) take this path with beta == 0 as well.
        const bool rd = beta_u != 0.0f;
        const TC* Ci = (const TC*)p.epi.cin + (sk ? 0 : (int64_t)b * p.epi.scin);
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            const int m = m0 + wm * WT + i * FR + fl;
            if (m < m_lo || m >= (int)p.M) continue;   // stored by the tile before an edge tile; past M
            TC* crow = Cb + (int64_t)m * p.ldc;
            const TC* cirow = Ci + (int64_t)m * p.epi.ldcin;
#pragma unroll
            for (int j = 0; j < NF; ++j) {
#pragma unroll
                for (int q = 0; q < NQ; ++q) {
                    const int n = n0 + wn * WT + j * FR + (SH == 0 ? 4 * (lane >> 4) : q * 8 + h * 4);
                    if (n < n_lo) continue;   // N % 4 == 0: a group of four is all below n_lo or none
                    float x[4], o[4] = {0.f, 0.f, 0.f, 0.f};
                    if (rd) load4<TC>(cirow + n, o, true);
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[e] = rd ? alpha * acc[i][j][q * 4 + e] + beta * o[e]
                                                          : alpha * acc[i][j][q * 4 + e];
                    if (has_bias) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) x[e] += bcol[j][q][e];
                    }
                    store4<TC>(crow + n, x, true);
                }
            }
        }
    }
    }
}

}  // namespace vkb
