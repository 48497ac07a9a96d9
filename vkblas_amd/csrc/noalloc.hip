// noalloc.hip — vkblas_gemm_noalloc_async: vkblas_gemm_async for callers
// that cannot allocate device memory (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc).  No counterpart in the
// reference.
//
// The only device memory vkblas_gemm_async allocates is the fp32 partials
// of split-K and of the split decode kernel ([split][M][N] floats).  Here
// they go to `scratch`, a file-scope device array of VKB_SCRATCH_BYTES that
// each GPU the library runs on holds from the code object's load until the
// process ends.  Host code never uses the array's name as an address (on the
// host it is only a stand-in symbol): the device address comes from
// hipGetSymbolAddress, taken once per device with that device current on
// the first call there, and kept per device.
//
// Every call on a device shares that device's array and finds it holding
// the previous call's partials.  The partials need no clearing: pass 1 of
// split-K and the decode kernel write every partial the reduce then reads.
// The array's first VKB_WS_HEADER bytes are the arrival counters of split-K
// passes that divide each K slice among workgroups; they must start at zero
// (each such launch then adds the same multiple to every counter it uses),
// so the first call on a device clears them with a fill kernel on its stream
// (no hipMemsetAsync: the call may be under stream capture).  Calls on one
// device that overlap in time (different streams, or different threads
// without ordering) race on the array; order them.
#include <hip/hip_runtime.h>
#include <pthread.h>
#include <stdint.h>

#include "vkb_engine.h"
#include "vkb_launch.h"
#include "vkblas_ext.h"

// 64 MiB of partials after the VKB_WS_HEADER bytes of arrival counters
#define VKB_SCRATCH_BYTES (((size_t)64 << 20) + VKB_WS_HEADER)

static __device__ __align__(256) unsigned char scratch[VKB_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
pthread_mutex_t g_scratch_lock = PTHREAD_MUTEX_INITIALIZER;
void* g_scratch_ptr[kMaxDevices];

__global__ void clear_words(uint32_t* p, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Device address of `scratch` on the current device (dev), or NULL.  The
// first call on a device also enqueues the clearing of the counters on
// `stream`, ahead of the call's own kernels.
void* scratch_on(int dev, hipStream_t stream) {
    pthread_mutex_lock(&g_scratch_lock);
    void* p = g_scratch_ptr[dev];
    if (!p) {
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) p = nullptr;
        if (p) {
            hipLaunchKernelGGL(clear_words, dim3(VKB_WS_COUNTERS / 256), dim3(256), 0, stream, (uint32_t*)p,
                               (uint32_t)VKB_WS_COUNTERS);
            if (hipGetLastError() != hipSuccess) p = nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    pthread_mutex_unlock(&g_scratch_lock);
    return p;
}

}  // namespace

extern "C" size_t vkblas_noalloc_scratch_bytes(void) { return VKB_SCRATCH_BYTES; }

extern "C" vkblas_status_t vkblas_gemm_noalloc_async(
    vkblas_dtype_t ab_type, vkblas_dtype_t c_type, vkblas_op_t op_a, vkblas_op_t op_b, uint32_t M, uint32_t N,
    uint32_t K, float alpha, const void* A, uint32_t lda, const void* B, uint32_t ldb, float beta, void* C,
    uint32_t ldc, uint32_t batch, int64_t stride_a, int64_t stride_b, int64_t stride_c,
    vkblas_scalar_mode_t scalar_mode, const void* alpha_dev, const void* beta_dev, uint32_t split_k,
    void* stream) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return VKBLAS_ERR_INIT;
    void* s = scratch_on(dev, (hipStream_t)stream);
    if (!s) return VKBLAS_ERR_INIT;
    return vkb_gemm_with_scratch(ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch,
                                 stride_a, stride_b, stride_c, scalar_mode, alpha_dev, beta_dev, split_k, stream, s,
                                 VKB_SCRATCH_BYTES);
}
