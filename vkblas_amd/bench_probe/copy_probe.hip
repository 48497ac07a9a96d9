// copy_probe.hip — the rate at which a CU copies GEMM operand tiles from L2
// into LDS by buffer_load ... lds (the pipelined GEMM kernel's copy path),
// with no compute.  Not a GEMM: it measures the ceiling the 16-bit GEMM
// kernels' operand copies are held to, and how it depends on the copies in
// flight and on the row segment each copy instruction covers.  No
// counterpart in the reference, and not part of libvkblas_hipblas.so: it
// builds into bench_probe/libvkblas_probe.so, which only bench.py and its
// test load.
//
// A and B are n x n fp16 matrices stored K-major (row r holds its n k
// contiguous), n a multiple of 256.  Workgroups are mapped to 256 x 256
// output tiles as the GEMM kernel maps them (gemm_pipe.hpp: with a grid of a
// multiple of 8 workgroups each XCD owns a contiguous run of tile indices,
// walked in groups of 4 tile rows), so each XCD's L2 serves the same operand
// panels as in the GEMM.  Workgroup b copies the K steps of its tile: per
// step the tile's 256 A rows and 256 B rows, RB bytes of
// each (RB 128: 64 k, one instruction per 8 rows, the GEMM kernel's shape;
// RB 64: 32 k, one instruction per 16 rows), into LDS stage step % 2.  D: the
// steps of copies in flight at each step's end (1: the step's own copies are
// waited for, as in a two-stage GEMM; 2: the next step's stay in flight).
// After the last step each workgroup writes the 32-bit wrapping sum of the
// words of its last stage, the copies of the last K step, to out[b].
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int RB>
struct CopyGeom {
    static constexpr int KS = RB / 2;                   // k per step
    static constexpr int RPI = 1024 / RB;               // rows per instruction
    static constexpr int NI = 64 / RPI;                 // instructions per operand, wave and step
    static constexpr int STAGE = 2 * 256 * RB / 16;     // 16-byte units per stage (A then B)
};

template <int D, int RB>
__global__ __launch_bounds__(256, 1) void copy_probe_kernel(const uint16_t* A, const uint16_t* B, uint32_t n,
                                                            uint32_t* out) {
    using G = CopyGeom<RB>;
    __shared__ u32x4 lds[2 * G::STAGE];
    __shared__ uint32_t red[256];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tiles = n / 256;
    uint32_t t = blockIdx.x;
    const uint32_t nwg = gridDim.x;
    if ((nwg & 7u) == 0) t = (t & 7u) * (nwg >> 3) + (t >> 3);
    const uint32_t width = 4 * tiles, group = t / width, first = 4 * group;
    const uint32_t gm = min(tiles - first, 4u), tin = t - group * width;
    const int m0 = (int)(first + tin % gm) * 256, n0 = (int)(tin / gm) * 256;
    const uint32_t bytes = n * n * 2u;
    auto rsrc = [&](const void* base) {
        const uint64_t a = (uint64_t)base;
        return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                     __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32) & 0xffff), (int)bytes, 0x00020000};
    };
    const i32x4 ra = rsrc(A), rb = rsrc(B);
    // lane l of instruction i: row 64 wave + RPI i + l / (RB / 16), chunk l % (RB / 16)
    constexpr int CPR = RB / 16;
    const int row = 64 * wave + lane / CPR;
    const int a_voff = (m0 + row) * (int)n * 2 + (lane % CPR) * 16;
    const int b_voff = (n0 + row) * (int)n * 2 + (lane % CPR) * 16;
    const int nkt = (int)n / G::KS;
    for (int kt = 0; kt < nkt; ++kt) {
        const int S = kt & 1;
#pragma unroll
        for (int op = 0; op < 2; ++op) {
#pragma unroll
            for (int i = 0; i < G::NI; ++i) {
                const int unit = S * G::STAGE + op * (G::STAGE / 2) + (G::NI * wave + i) * 64;
                const int m0r = __builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(
                    __attribute__((address_space(3))) void*)&lds[unit]);
                const int soff = __builtin_amdgcn_readfirstlane((kt * G::KS + G::RPI * i * (int)n) * 2);
                asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds"
                             :: "v"(op ? b_voff : a_voff), "s"(op ? rb : ra), "s"(soff), "{m0}"(m0r)
                             : "memory");
            }
        }
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(2 * G::NI * (D - 1)) : "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    // checksum of the last stage (the copies of step nkt - 1)
    const u32x4* st = lds + ((nkt - 1) & 1) * G::STAGE;
    uint32_t s = 0;
    for (int u = threadIdx.x; u < G::STAGE; u += 256) {
        const u32x4 v = st[u];
        s += v[0] + v[1] + v[2] + v[3];
    }
    red[threadIdx.x] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t total = 0;
        for (int i = 0; i < 256; ++i) total += red[i];
        out[blockIdx.x] = total;
    }
}

}  // namespace

// steps_in_flight 1 or 2, row_bytes 128 or 64, blocks <= (n / 256)^2, n a
// multiple of 256 up to 16384; A, B 16-byte aligned, out 4-byte aligned.
extern "C" int vkblas_copy_probe(const void* A, const void* B, uint32_t n, uint32_t blocks, int steps_in_flight,
                                 int row_bytes, uint32_t* out, void* stream) {
    if (!A || !B || !out || n == 0 || n % 256 != 0 || n > 16384 || blocks == 0 ||
        blocks > (n / 256) * (n / 256) || (steps_in_flight != 1 && steps_in_flight != 2) ||
        (row_bytes != 128 && row_bytes != 64) || ((uintptr_t)A & 15) || ((uintptr_t)B & 15) ||
        ((uintptr_t)out & 3))
        return (int)hipErrorInvalidValue;
    hipStream_t st = (hipStream_t)stream;
    const uint16_t* a = (const uint16_t*)A;
    const uint16_t* b = (const uint16_t*)B;
    if (row_bytes == 128) {
        if (steps_in_flight == 1)
            hipLaunchKernelGGL((copy_probe_kernel<1, 128>), dim3(blocks), dim3(256), 0, st, a, b, n, out);
        else
            hipLaunchKernelGGL((copy_probe_kernel<2, 128>), dim3(blocks), dim3(256), 0, st, a, b, n, out);
    } else {
        if (steps_in_flight == 1)
            hipLaunchKernelGGL((copy_probe_kernel<1, 64>), dim3(blocks), dim3(256), 0, st, a, b, n, out);
        else
            hipLaunchKernelGGL((copy_probe_kernel<2, 64>), dim3(blocks), dim3(256), 0, st, a, b, n, out);
    }
    return (int)hipGetLastError();
}
