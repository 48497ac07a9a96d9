// gemm_mfma.hpp — blocked MFMA GEMM for gfx950 (CDNA4), fp32, fp16 and bf16 inputs.
//
// Replaces the reference's tiled GLSL GEMMs (gemm_f32_128x128_bankfree_tmpl.comp,
// gemm_half_128x128_bankfree_tmpl.comp and their 64x64 / 128x256 / split-K
// siblings, dispatched from src/vkblas.c:1191-1313, 1759-1868, 1873-2096) and the
// host-side transpose pass the reference ran in front of them
// (src/vkblas.c:972-1105, 1333-1475): every TA/TB variant is read natively.
//
// Design (one workgroup = 4 waves of 64 lanes, 2x2 wave grid):
//  * LDS holds both operand tiles K-contiguous: tile row r (an m of A or an
//    n of B) is 128 bytes of K (32 fp32 / 64 fp16) split in eight 16-byte
//    chunks.  Chunk c of row r lives at slot c ^ ((r ^ (r >> 3)) & 7).  With
//    that XOR swizzle the three access patterns — K-major global rows written
//    8 chunks per row, MN-major sub-blocks written one row per lane 8 (or 4)
//    rows apart, and MFMA operand reads of 32 consecutive rows at one chunk —
//    all hit distinct 16-byte bank groups within every 8 lanes, with no padding.
//  * A K-major operand (A with op_a = N, B with op_b = T) streams global->LDS
//    as 16-byte vectors.  An MN-major operand is loaded as VEC k-rows x VEC
//    consecutive m (or n), transposed in registers (free for fp32: register
//    renaming; v_perm for fp16) and written as K-contiguous 16-byte chunks.
//  * MFMA roles are swapped: src A = B tile (rows n), src B = A tile (rows m),
//    so D = C^T per 32x32 tile and each lane owns 4 consecutive n of one row m
//    of C: the epilogue stores 16 B (fp32) or 8 B (fp16) per lane.
//  * Two LDS stages; global loads for tile k+1 are issued before the MFMAs of
//    tile k and land in registers; one barrier per K step.
//  * Workgroup ids are remapped so each XCD (ids are dealt round-robin over
//    the 8 XCDs) owns a contiguous run of tiles, and tiles are visited in
//    groups of 8 tile-rows so neighbours share A rows and B columns in L2.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "epilogue.hpp"

namespace vkb {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct KParams {
    const void* A;
    const void* B;
    void* C;
    int64_t lda, ldb, ldc;
    int64_t sa, sb, sc;     // batch strides (elements)
    int64_t s_split;        // split-K partial stride in C (elements)
    uint32_t M, N, K;
    uint32_t tiles_m, tiles_n;
    uint32_t split, kps;
    uint32_t batch;
    float alpha, beta;
    const void* alpha_dev;
    const void* beta_dev;
    int scalar_mode;
    int vec_a, vec_b, vec_c;
    // every C row starts 16-byte aligned (ldc * sizeof(TC) % 16 == 0, C, the
    // batch stride and the split-K stride too): the pipelined kernel's
    // staged epilogue stores whole rows in 16-byte units
    int c_rows16;
    // Cin (beta's matrix) and the bias vector; vec_c covers Cin's alignment too
    EpiParams epi;
    // A, B, C are device arrays of `batch` matrix pointers (the sa / sb / sc
    // strides are unused); vec_* then also need each matrix aligned, which
    // the kernel checks per batch
    int ptr_array;
    // wave-K split-K pass 1 with each K slice over nq workgroups (nq > 1):
    // their sums in qpart, their arrival counters in qcnt
    uint32_t nq;
    float* qpart;
    uint32_t* qcnt;
};

template <typename T> struct Elem;
template <> struct Elem<float>    { static constexpr int VEC = 4; static constexpr int BK = 32; };
template <> struct Elem<_Float16> { static constexpr int VEC = 8; static constexpr int BK = 64; };
template <> struct Elem<__bf16>   { static constexpr int VEC = 8; static constexpr int BK = 64; };

template <typename T> constexpr bool is_bf16 = __is_same(T, __bf16);

// 16-bit MFMAs on raw 16-byte fragments (8 elements of k per lane): fp16 or
// bf16 by the element type.  srcA / srcB order as the hardware takes them.
template <typename T>
__device__ __forceinline__ floatx16 mfma_32x32x16(u32x4 a, u32x4 b, floatx16 c) {
    if constexpr (is_bf16<T>)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a),
                                                      __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
}

template <typename T>
__device__ __forceinline__ floatx4 mfma_16x16x32(u32x4 a, u32x4 b, floatx4 c) {
    if constexpr (is_bf16<T>)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                      __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
}

__device__ __forceinline__ int swz(int row, int chunk) {
    return chunk ^ ((row ^ (row >> 3)) & 7);
}

__device__ __forceinline__ void load_scalars(const KParams& p, float& alpha, float& beta) {
    alpha = p.alpha;
    beta = p.beta;
    if (p.scalar_mode == 1) {
        alpha = *(const float*)p.alpha_dev;
        beta = *(const float*)p.beta_dev;
    } else if (p.scalar_mode == 2) {
        alpha = (float)*(const _Float16*)p.alpha_dev;
        beta = (float)*(const _Float16*)p.beta_dev;
    }
}

// one element as raw bits, zero when out of range
template <typename T>
__device__ __forceinline__ uint32_t ld_bits(const T* p, bool ok) {
    if constexpr (sizeof(T) == 4) {
        return ok ? *(const uint32_t*)p : 0u;
    } else {
        return ok ? (uint32_t)(*(const uint16_t*)p) : 0u;
    }
}

// VEC consecutive elements, element i valid iff ok && i < nvalid
template <typename T>
__device__ __forceinline__ u32x4 ld_vec_checked(const T* p, bool ok, int nvalid, bool vec_ok) {
    constexpr int VEC = Elem<T>::VEC;
    if (ok && vec_ok && nvalid >= VEC) return *(const u32x4*)p;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (ok) {
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = ld_bits(p + i, i < nvalid);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) w[i >> 1] |= ld_bits(p + i, i < nvalid) << (16 * (i & 1));
        }
    }
    return u32x4{w[0], w[1], w[2], w[3]};
}

// Row i of the transpose of a VEC x VEC block held as VEC vectors (one per k).
template <typename T>
__device__ __forceinline__ u32x4 transpose_row(const u32x4* v, int i) {
    if constexpr (sizeof(T) == 4) {
        return u32x4{v[0][i], v[1][i], v[2][i], v[3][i]};
    } else {
        uint32_t o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t lo = v[2 * j][i >> 1];
            const uint32_t hi = v[2 * j + 1][i >> 1];
            o[j] = (i & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
        return u32x4{o[0], o[1], o[2], o[3]};
    }
}

// Global -> register -> LDS staging of one operand tile: R rows (m or n) x BK.
template <typename T, int R, bool KMAJ, bool CHECKED>
struct Stager {
    static constexpr int VEC = Elem<T>::VEC;
    static constexpr int BK = Elem<T>::BK;
    // K-major: R*8 16-byte chunks.  MN-major: 8*(R/VEC) VECxVEC blocks.
    static constexpr int NCHUNK = R * 8;
    static constexpr int NBLK = 8 * (R / VEC);
    static constexpr int NV = KMAJ ? (NCHUNK + 255) / 256 : ((NBLK + 255) / 256) * VEC;
    u32x4 v[NV];

    // base: operand pointer for this batch; row0: first m/n of the tile;
    // rows: M or N; k0: first k of this K step; kend: end of this K slice.
    __device__ __forceinline__ void load(const T* base, int64_t ld, int row0, int rows, int k0,
                                         int kend, bool vec_ok, int tid) {
        if constexpr (KMAJ) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int c = tid + i * 256;
                if (NCHUNK % 256 == 0 || c < NCHUNK) {
                    const int r = c >> 3, kc = c & 7;
                    const int row = row0 + r, k = k0 + kc * VEC;
                    const T* ptr = base + (int64_t)row * ld + k;
                    if constexpr (!CHECKED) {
                        v[i] = *(const u32x4*)ptr;
                    } else {
                        v[i] = ld_vec_checked<T>(ptr, row < rows, kend - k, vec_ok);
                    }
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < NV / VEC; ++j) {
                const int bi = tid + j * 256;
                if (NBLK % 256 == 0 || bi < NBLK) {
                    const int kb = bi / (R / VEC), mb = bi % (R / VEC);
                    const int mn = row0 + mb * VEC;
#pragma unroll
                    for (int kk = 0; kk < VEC; ++kk) {
                        const int k = k0 + kb * VEC + kk;
                        const T* ptr = base + (int64_t)k * ld + mn;
                        if constexpr (!CHECKED) {
                            v[j * VEC + kk] = *(const u32x4*)ptr;
                        } else {
                            v[j * VEC + kk] = ld_vec_checked<T>(ptr, k < kend, rows - mn, vec_ok);
                        }
                    }
                }
            }
        }
    }

    __device__ __forceinline__ void store(u32x4* tile, int tid) const {
        if constexpr (KMAJ) {
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int c = tid + i * 256;
                if (NCHUNK % 256 == 0 || c < NCHUNK) {
                    const int r = c >> 3, kc = c & 7;
                    tile[r * 8 + swz(r, kc)] = v[i];
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < NV / VEC; ++j) {
                const int bi = tid + j * 256;
                if (NBLK % 256 == 0 || bi < NBLK) {
                    const int kb = bi / (R / VEC), mb = bi % (R / VEC);
#pragma unroll
                    for (int i = 0; i < VEC; ++i) {
                        const int r = mb * VEC + i;
                        tile[r * 8 + swz(r, kb)] = transpose_row<T>(&v[j * VEC], i);
                    }
                }
            }
        }
    }
};

// Four results to C: fp32 as is, fp16 / bf16 rounded to nearest even.
template <typename TC>
__device__ __forceinline__ void store4(TC* p, const float* x, bool vec) {
    if constexpr (sizeof(TC) == 4) {
        if (vec) {
            *(float4*)p = make_float4(x[0], x[1], x[2], x[3]);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = x[i];
        }
    } else {
        typedef TC v4 __attribute__((ext_vector_type(4)));
        if (vec) {
            v4 h;
            h[0] = (TC)x[0]; h[1] = (TC)x[1];
            h[2] = (TC)x[2]; h[3] = (TC)x[3];
            *(v4*)p = h;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) p[i] = (TC)x[i];
        }
    }
}

template <typename TC>
__device__ __forceinline__ void load4(const TC* p, float* x, bool vec) {
    if constexpr (sizeof(TC) == 4) {
        if (vec) {
            float4 f = *(const float4*)p;
            x[0] = f.x; x[1] = f.y; x[2] = f.z; x[3] = f.w;
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = p[i];
        }
    } else {
        typedef TC v4 __attribute__((ext_vector_type(4)));
        if (vec) {
            v4 h = *(const v4*)p;
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = (float)h[i];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = (float)p[i];
        }
    }
}

// T: input element, TC: output element, AK: A is K-major (op_a == N),
// BKM: B is K-major (op_b == T), BM x BN block tile, CHECKED: edge handling.
template <typename T, typename TC, bool AK, bool BKM, int BM, int BN, bool CHECKED>
__global__ __launch_bounds__(256) void gemm_kernel(KParams p) {
    constexpr int BK = Elem<T>::BK;
    constexpr int WTM = BM / 2, WTN = BN / 2;   // wave tile
    constexpr int TM = WTM / 32, TN = WTN / 32; // 32x32 MFMA tiles per wave
    __shared__ u32x4 lds[2][(BM + BN) * 8];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int l32 = lane & 31, h = lane >> 5;

    // ---- tile / batch / split decode with XCD-aware remap ----
    uint32_t bid = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if ((nwg & 7u) == 0) bid = (bid & 7u) * (nwg >> 3) + (bid >> 3);
    const uint32_t per = p.tiles_m * p.tiles_n;
    const uint32_t z = bid / per;
    const uint32_t t = bid - z * per;
    const uint32_t b = z / p.split;
    const uint32_t s = z - b * p.split;
    constexpr uint32_t GM = 8;
    const uint32_t width = GM * p.tiles_n;
    const uint32_t group = t / width;
    const uint32_t first_m = group * GM;
    const uint32_t gm = min(p.tiles_m - first_m, GM);
    const uint32_t tin = t - group * width;
    const int m0 = (int)(first_m + tin % gm) * BM;
    const int n0 = (int)(tin / gm) * BN;

    const T* Ab;
    const T* Bb;
    TC* Cb;
    const TC* Ci;   // beta's matrix (Cb itself in place)
    bool va = p.vec_a != 0, vb = p.vec_b != 0, vc = p.vec_c != 0;
    if (p.ptr_array) {
        Ab = ((const T* const*)p.A)[b];
        Bb = ((const T* const*)p.B)[b];
        Cb = ((TC* const*)p.C)[b];
        Ci = Cb;
        va = va && ((uintptr_t)Ab & 15) == 0;
        vb = vb && ((uintptr_t)Bb & 15) == 0;
        vc = vc && ((uintptr_t)Cb & (4 * sizeof(TC) - 1)) == 0;
    } else {
        Ab = (const T*)p.A + (int64_t)b * p.sa;
        Bb = (const T*)p.B + (int64_t)b * p.sb;
        Cb = (TC*)p.C + (int64_t)b * p.sc + (int64_t)s * p.s_split;
        Ci = (const TC*)p.epi.cin + (int64_t)b * p.epi.scin;
    }
    const int64_t ldci = p.ptr_array ? p.ldc : p.epi.ldcin;
    const int kbeg = (int)(s * p.kps);
    const int kend = (int)min((uint32_t)p.K, s * p.kps + p.kps);
    const int nkt = (kend - kbeg + BK - 1) / BK;

    Stager<T, BM, AK, CHECKED> sa;
    Stager<T, BN, BKM, CHECKED> sb;

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    if (nkt > 0) {
        sa.load(Ab, p.lda, m0, (int)p.M, kbeg, kend, va, tid);
        sb.load(Bb, p.ldb, n0, (int)p.N, kbeg, kend, vb, tid);
        sa.store(&lds[0][0], tid);
        sb.store(&lds[0][BM * 8], tid);
    }
    __syncthreads();

    // LDS rows this lane reads for its MFMA operands
    int arow[TM], brow[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) arow[i] = wm * WTM + i * 32 + l32;
#pragma unroll
    for (int j = 0; j < TN; ++j) brow[j] = wn * WTN + j * 32 + l32;

    for (int kt = 0; kt < nkt; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nkt;
        if (more) {
            const int k0 = kbeg + (kt + 1) * BK;
            sa.load(Ab, p.lda, m0, (int)p.M, k0, kend, va, tid);
            sb.load(Bb, p.ldb, n0, (int)p.N, k0, kend, vb, tid);
        }
        const u32x4* As = &lds[cur][0];
        const u32x4* Bs = &lds[cur][BM * 8];
        if constexpr (sizeof(T) == 2) {
            // v_mfma_f32_32x32x16_f16: lane holds 8 k of one row; step st covers
            // k in [16 st, 16 st + 16), lane half h takes the upper 8.
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int c = 2 * st + h;
                u32x4 af[TM], bf[TN];
#pragma unroll
                for (int j = 0; j < TN; ++j) bf[j] = Bs[brow[j] * 8 + swz(brow[j], c)];
#pragma unroll
                for (int i = 0; i < TM; ++i) af[i] = As[arow[i] * 8 + swz(arow[i], c)];
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = mfma_32x32x16<T>(bf[j], af[i], acc[i][j]);
            }
        } else {
            // v_mfma_f32_32x32x2_f32: lane holds 1 k of one row.  Lane half h
            // owns k in [16 h, 16 h + 16) of the 32-wide step, one per MFMA.
            // Fragments are double-buffered: the reads of chunk q+1 are issued
            // before the 4 TM TN MFMAs of chunk q, so LDS latency stays hidden.
            // Each read is fenced (sched_barrier) between groups of MFMAs so the
            // compiler cannot sink it next to its first use.
            constexpr int NF = TM + TN;                 // fragment reads per chunk
            constexpr int NM = 4 * TM * TN;             // MFMAs per chunk
            u32x4 af[2][TM], bf[2][TN];
            auto read_frag = [&](int q, int buf, int f) {
                const int c = h * 4 + q;
                if (f < TN) bf[buf][f] = Bs[brow[f] * 8 + swz(brow[f], c)];
                else af[buf][f - TN] = As[arow[f - TN] * 8 + swz(arow[f - TN], c)];
            };
#pragma unroll
            for (int f = 0; f < NF; ++f) read_frag(0, 0, f);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
#pragma unroll
                for (int u = 0; u < NM; ++u) {
                    const int e = u / (TM * TN), i = (u / TN) % TM, j = u % TN;
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(bf[q & 1][j][e]),
                                                                    __uint_as_float(af[q & 1][i][e]), acc[i][j],
                                                                    0, 0, 0);
                    if (q < 3 && u % (NM / NF) == 0) read_frag(q + 1, (q + 1) & 1, u / (NM / NF));
                    if (u % (NM / NF) == NM / NF - 1) __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        if (more) {
            sa.store(&lds[cur ^ 1][0], tid);
            sb.store(&lds[cur ^ 1][BM * 8], tid);
        }
        __syncthreads();
    }

    // ---- epilogue: C[m][n..n+3] = alpha * acc + beta * C ----
    float alpha, beta;
    load_scalars(p, alpha, beta);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int m = m0 + wm * WTM + i * 32 + l32;
        if (CHECKED && m >= (int)p.M) continue;
        TC* crow = Cb + (int64_t)m * p.ldc;
        const TC* cirow = Ci + (int64_t)m * ldci;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wn * WTN + j * 32 + q * 8 + h * 4;
                float x[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) x[e] = alpha * acc[i][j][q * 4 + e];
                if constexpr (!CHECKED) {
                    if (beta != 0.0f) {
                        float o[4];
                        load4<TC>(cirow + n, o, true);
#pragma unroll
                        for (int e = 0; e < 4; ++e) x[e] += beta * o[e];
                    }
                    add_bias4(p.epi, n, 4, x);
                    store4<TC>(crow + n, x, true);
                } else {
                    const int nv = (int)p.N - n;
                    if (nv >= 4) {
                        if (beta != 0.0f) {
                            float o[4];
                            load4<TC>(cirow + n, o, vc);
#pragma unroll
                            for (int e = 0; e < 4; ++e) x[e] += beta * o[e];
                        }
                        add_bias4(p.epi, n, 4, x);
                        store4<TC>(crow + n, x, vc);
                    } else {
                        if (beta != 0.0f) {
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                if (e < nv) x[e] += beta * (float)cirow[n + e];
                        }
                        add_bias4(p.epi, n, nv, x);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (e < nv) crow[n + e] = (TC)x[e];
                    }
                }
            }
        }
    }
}

}  // namespace vkb
