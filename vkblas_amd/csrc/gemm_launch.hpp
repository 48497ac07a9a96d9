// gemm_launch.hpp — host-side launcher for gemm_kernel<> (one instantiation
// set per element-type pair; gemm_f32.hip / gemm_f16.hip include this).
#pragma once
#include "gemm_mfma.hpp"
#include "gemm_pipe.hpp"
#include "gemm_wavek.hpp"
#include "vkb_launch.h"

namespace vkb {

template <int TILE> struct TileDim;
template <> struct TileDim<VKB_TILE_64>  { static constexpr int BM = 64,  BN = 64;  };
template <> struct TileDim<VKB_TILE_128> { static constexpr int BM = 128, BN = 128; };
template <> struct TileDim<VKB_TILE_256> { static constexpr int BM = 256, BN = 256; };

template <typename T, typename TC, bool AK, bool BKM, int TILE, bool CHECKED>
static int launch_one(const KParams& p, uint32_t grid, hipStream_t st) {
    constexpr int BM = TileDim<TILE>::BM, BN = TileDim<TILE>::BN;
    hipLaunchKernelGGL((gemm_kernel<T, TC, AK, BKM, BM, BN, CHECKED>), dim3(grid), dim3(256), 0, st, p);
    return (int)hipGetLastError();
}

template <typename T, typename TC, bool AK, bool BKM, int TILE>
static int launch_ck(const KParams& p, bool checked, uint32_t grid, hipStream_t st) {
    return checked ? launch_one<T, TC, AK, BKM, TILE, true>(p, grid, st)
                   : launch_one<T, TC, AK, BKM, TILE, false>(p, grid, st);
}

template <typename T, typename TC, int TILE>
static int launch_layout(const KParams& p, bool ak, bool bk, bool checked, uint32_t grid, hipStream_t st) {
    if (ak) {
        return bk ? launch_ck<T, TC, true, true, TILE>(p, checked, grid, st)
                  : launch_ck<T, TC, true, false, TILE>(p, checked, grid, st);
    }
    return bk ? launch_ck<T, TC, false, true, TILE>(p, checked, grid, st)
              : launch_ck<T, TC, false, false, TILE>(p, checked, grid, st);
}

static inline bool aligned(const void* ptr, uintptr_t a) { return ((uintptr_t)ptr % a) == 0; }

// Compute units of the current device (cached per device; 0 if unknown).
static inline uint32_t cu_count() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int n = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 0) n = 0;
        __atomic_store_n(&cached[dev], n, __ATOMIC_RELAXED);
    }
    return (uint32_t)n;
}

// Bytes of K per step of the wave-K kernel for 16-bit inputs: 128 (whole
// 128-byte rows of a K-major operand per copy).  Measured against 64 (more
// stages of half rows), M = N = 256, fp16, hipBLAS NN, split 4 / 16: K =
// 65536 45.4 / 24.1 -> 36.7 / 19.8 us, K = 262144 163.5 / 83.1 -> 133.5 /
// 66.5 us (two alternating runs, one box).
#ifndef VKB_WAVEK_KB16
#define VKB_WAVEK_KB16 128
#endif
constexpr int WK_KB16 = VKB_WAVEK_KB16;

template <typename T, typename TC>
static int launch_gemm_typed(const vkb_gemm_args* a, int tile, hipStream_t st) {
    constexpr int VEC = Elem<T>::VEC;
    constexpr int BK = Elem<T>::BK;
    static_assert(WAVEK_NQ == VKB_WAVEK_NQ, "one part count");
    int bm = 64, bn = 64;
    if (tile == VKB_TILE_128) { bm = bn = 128; }
    else if (tile == VKB_TILE_256) { bm = bn = 256; }
    else if (tile == VKB_TILE_32) { bm = bn = 32; }
    else if (tile != VKB_TILE_64 && tile != VKB_TILE_64Q) return (int)hipErrorInvalidValue;

    KParams p{};
    p.A = a->A; p.B = a->B; p.C = a->C;
    p.lda = a->lda; p.ldb = a->ldb; p.ldc = a->ldc;
    p.sa = a->stride_a; p.sb = a->stride_b; p.sc = a->stride_c;
    p.M = a->M; p.N = a->N; p.K = a->K;
    p.batch = a->batch ? a->batch : 1;
    p.split = a->split > 1 ? a->split : 1;
    p.kps = p.split > 1 ? a->k_per_split : a->K;
    p.s_split = p.split > 1 ? a->stride_split : 0;
    p.tiles_m = (a->M + bm - 1) / bm;
    p.tiles_n = (a->N + bn - 1) / bn;
    p.alpha = a->alpha; p.beta = a->beta;
    p.scalar_mode = a->scalar_mode;
    p.alpha_dev = a->alpha_dev; p.beta_dev = a->beta_dev;
    const vkb_epilogue_args* ep = a->epi;
    const bool sep_cin = ep && ep->c_in && p.split == 1;   // pass 1 writes raw partials
    p.epi.cin = sep_cin ? ep->c_in : a->C;
    p.epi.ldcin = sep_cin ? ep->ldc_in : a->ldc;
    p.epi.scin = sep_cin ? ep->stride_c_in : a->stride_c;
    p.epi.bias = (ep && p.split == 1) ? ep->bias : nullptr;
    p.epi.bias_type = ep ? ep->bias_type : 0;
    p.ptr_array = a->ptr_array != 0;
    if (p.ptr_array && sep_cin) return (int)hipErrorInvalidValue;   // Cin pointers are not given
    // each K slice over VKB_WAVEK_NQ workgroups: the wave-K kernel only (below)
    p.nq = tile == VKB_TILE_64Q ? VKB_WAVEK_NQ : 1;
    p.qpart = a->qpart;
    p.qcnt = a->qcnt;
    if (tile == VKB_TILE_64Q &&
        (p.split < 2 || p.ptr_array || !a->qpart || !a->qcnt || ((uintptr_t)a->qpart & 15) ||
         ((uintptr_t)a->qcnt & 3) || (uint64_t)p.split * p.tiles_m * p.tiles_n > VKB_WS_COUNTERS))
        return (int)hipErrorInvalidValue;
    const bool multi = p.batch > 1;
    if (p.ptr_array) {
        // the matrices' alignment is checked per batch in the kernel, which
        // always runs the checked instantiation (no pipelined kernel)
        if (p.split > 1) return (int)hipErrorInvalidValue;
        p.vec_a = a->lda % VEC == 0;
        p.vec_b = a->ldb % VEC == 0;
        p.vec_c = a->ldc % 4 == 0;
    } else {
        p.vec_a = (a->lda % VEC == 0) && aligned(a->A, 16) && (!multi || a->stride_a % VEC == 0);
        p.vec_b = (a->ldb % VEC == 0) && aligned(a->B, 16) && (!multi || a->stride_b % VEC == 0);
        p.vec_c = (a->ldc % 4 == 0) && aligned(a->C, 4 * sizeof(TC)) && (!multi || a->stride_c % 4 == 0) &&
                  (p.split == 1 || p.s_split % 4 == 0);
        if (sep_cin)   // Cin is read with the same vector width as C
            p.vec_c = p.vec_c && p.epi.ldcin % 4 == 0 && aligned(p.epi.cin, 4 * sizeof(TC)) &&
                      (!multi || p.epi.scin % 4 == 0);
    }
    {
        constexpr int64_t CV = 16 / sizeof(TC);   // elements per 16 bytes of C
        // an edge tile (N not a multiple of the tile) stores from a shifted
        // column N - BN on: whole 16-byte chunks need N % CV == 0 as well
        p.c_rows16 = !p.ptr_array && a->ldc % CV == 0 && aligned(a->C, 16) && (!multi || a->stride_c % CV == 0) &&
                     (p.split == 1 || p.s_split % CV == 0) && (a->N % bn == 0 || a->N % CV == 0);
    }
    auto report = [&](int k) {
        if (a->kernel_out) *a->kernel_out = k;
    };
    if (p.split > 1 && (p.kps == 0 || p.kps % BK != 0)) return (int)hipErrorInvalidValue;

    const bool full = !p.ptr_array && (a->M % bm == 0) && (a->N % bn == 0) && (a->K % BK == 0) &&
                      p.vec_a && p.vec_b && p.vec_c;
    const uint64_t grid64 = (uint64_t)p.tiles_m * p.tiles_n * p.batch * p.split * p.nq;
    if (grid64 == 0 || grid64 > 0x7fffffffull) return (int)hipErrorInvalidValue;
    const uint32_t grid = (uint32_t)grid64;
    const bool ak = a->a_kmajor != 0, bk = a->b_kmajor != 0;
    {
        // software-pipelined kernel for full 256x256 and 128x128 tiles (also
        // split-K pass 1 on them).  K and the split-K slice a multiple of two
        // K steps (128 bytes each): the loop runs pairs.  Buffer offsets are
        // signed 32-bit: bound the byte span of each operand tile.
        // Edge tiles (M or N not a multiple of the tile) shift back inside
        // the matrix: M >= bm, N >= bn; the shifted start of an MN-major
        // operand stays 16-byte aligned (M or N a multiple of VEC); the
        // epilogue masks groups of four columns (N % 4 == 0).
        constexpr uint64_t ES = sizeof(T);
        constexpr uint32_t KPAIR = 256 / sizeof(T);
        const uint64_t span_a = ((uint64_t)(a->a_kmajor ? bm : a->K) * (uint64_t)a->lda + a->K) * ES;
        const uint64_t span_b = ((uint64_t)(a->b_kmajor ? bn : a->K) * (uint64_t)a->ldb + a->K) * ES;
        // M < bm: 128x128 tiles with K-major A (rows past M read as row M - 1)
        const bool edges_ok = (a->M >= (uint32_t)bm || (bm == 128 && ak)) && a->N >= (uint32_t)bn && a->N % 4 == 0 &&
                              (a->a_kmajor || a->M % VEC == 0) && (a->b_kmajor || a->N % VEC == 0);
        const bool tiles_ok = !p.ptr_array && (a->K % BK == 0) && p.vec_a && p.vec_b && p.vec_c &&
                              (full || edges_ok);
        const bool pipe_ok = tiles_ok && (p.split == 1 || p.kps % KPAIR == 0) && !a->generic_only &&
                             a->K % KPAIR == 0 && span_a < (1ull << 31) && span_b < (1ull << 31);
        if (tile == VKB_TILE_256 && pipe_ok) {
            report(VKB_KERN_PIPE256);
            if (ak) {
                if (bk) hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, true, true>), dim3(grid), dim3(256), 0, st, p);
                else hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, true, false>), dim3(grid), dim3(256), 0, st, p);
            } else {
                if (bk) hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, false, true>), dim3(grid), dim3(256), 0, st, p);
                else hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, false, false>), dim3(grid), dim3(256), 0, st, p);
            }
            return (int)hipGetLastError();
        }
        // 128x128 tiles: the pipelined kernel with 64x64 wave tiles.  16-bit
        // types take four LDS stages when the grid is at most one workgroup
        // per CU (the 144 KB they take allow no second one), else two; fp32
        // (a K step is 4096 MFMA cycles, longer than the load latency) always
        // two.
        if (tile == VKB_TILE_128 && pipe_ok) {
            const bool four = sizeof(T) == 2 && grid <= cu_count();
            report(four ? VKB_KERN_PIPE128_4 : VKB_KERN_PIPE128);
            if constexpr (sizeof(T) == 2) {
                if (four) {
                    if (ak) {
                        if (bk) hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, true, true, 64, 4>), dim3(grid), dim3(256), 0, st, p);
                        else hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, true, false, 64, 4>), dim3(grid), dim3(256), 0, st, p);
                    } else {
                        if (bk) hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, false, true, 64, 4>), dim3(grid), dim3(256), 0, st, p);
                        else hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, false, false, 64, 4>), dim3(grid), dim3(256), 0, st, p);
                    }
                    return (int)hipGetLastError();
                }
            }
            if (ak) {
                if (bk) hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, true, true, 64>), dim3(grid), dim3(256), 0, st, p);
                else hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, true, false, 64>), dim3(grid), dim3(256), 0, st, p);
            } else {
                if (bk) hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, false, true, 64>), dim3(grid), dim3(256), 0, st, p);
                else hipLaunchKernelGGL((gemm_pipe_kernel<T, TC, false, false, 64>), dim3(grid), dim3(256), 0, st, p);
            }
            return (int)hipGetLastError();
        }
    }
    // Split-K pass 1 on 32x32 or 64x64 tiles (few output tiles, a caller's
    // split): the wave-K kernel, whose four waves each take a quarter of the
    // slice's K.  Whole tiles, K and the slice in whole K steps, aligned
    // operands; buffer offsets are signed 32-bit.
    if constexpr (std::is_same<TC, float>::value) {
        if ((tile == VKB_TILE_32 || tile == VKB_TILE_64 || tile == VKB_TILE_64Q) && p.split > 1 && !p.ptr_array &&
            !a->generic_only) {
            constexpr uint64_t ES = sizeof(T);
            const uint32_t tt = (uint32_t)bm;
            const uint64_t span_a = ((uint64_t)(ak ? tt : a->K) * (uint64_t)a->lda + a->K) * ES;
            const uint64_t span_b = ((uint64_t)(bk ? tt : a->K) * (uint64_t)a->ldb + a->K) * ES;
            constexpr uint32_t KS = sizeof(T) == 2 ? WK_KB16 / 2 : 32;   // k per step
            if (a->M % tt == 0 && a->N % tt == 0 && a->K % KS == 0 && p.kps % KS == 0 && p.vec_a && p.vec_b &&
                p.vec_c && span_a < (1ull << 31) && span_b < (1ull << 31)) {
                report(VKB_KERN_WAVEK);
                if (tt == 32) {
                    if (ak) {
                        if (bk) hipLaunchKernelGGL((gemm_wavek_kernel<T, true, true, 32, WK_KB16>), dim3(grid), dim3(256), 0, st, p);
                        else hipLaunchKernelGGL((gemm_wavek_kernel<T, true, false, 32, WK_KB16>), dim3(grid), dim3(256), 0, st, p);
                    } else {
                        if (bk) hipLaunchKernelGGL((gemm_wavek_kernel<T, false, true, 32, WK_KB16>), dim3(grid), dim3(256), 0, st, p);
                        else hipLaunchKernelGGL((gemm_wavek_kernel<T, false, false, 32, WK_KB16>), dim3(grid), dim3(256), 0, st, p);
                    }
                } else {
                    if (ak) {
                        if (bk) hipLaunchKernelGGL((gemm_wavek_kernel<T, true, true, 64, WK_KB16>), dim3(grid), dim3(256), 0, st, p);
                        else hipLaunchKernelGGL((gemm_wavek_kernel<T, true, false, 64, WK_KB16>), dim3(grid), dim3(256), 0, st, p);
                    } else {
                        if (bk) hipLaunchKernelGGL((gemm_wavek_kernel<T, false, true, 64, WK_KB16>), dim3(grid), dim3(256), 0, st, p);
                        else hipLaunchKernelGGL((gemm_wavek_kernel<T, false, false, 64, WK_KB16>), dim3(grid), dim3(256), 0, st, p);
                    }
                }
                return (int)hipGetLastError();
            }
        }
    }
    // only the wave-K kernel takes 32x32 tiles or divided slices
    if (tile == VKB_TILE_32 || tile == VKB_TILE_64Q) return (int)hipErrorInvalidValue;
    report(full ? VKB_KERN_GENERIC : VKB_KERN_GENERIC_CHECKED);
    switch (tile) {
        case VKB_TILE_64:  return launch_layout<T, TC, VKB_TILE_64>(p, ak, bk, !full, grid, st);
        case VKB_TILE_128: return launch_layout<T, TC, VKB_TILE_128>(p, ak, bk, !full, grid, st);
        default:           return launch_layout<T, TC, VKB_TILE_256>(p, ak, bk, !full, grid, st);
    }
}

}  // namespace vkb
