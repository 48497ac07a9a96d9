/*
 * engine_stub.c — the public C API of libvkblas_hipblas.so (include/vkblas.h,
 * include/vkblas_ext.h), forwarded to libvkblas_engine.so, the host
 * dispatcher and gfx950 kernels, which is loaded from this library's own
 * directory at the first call.
 *
 * Why two libraries.  The reference is used as
 * `LD_PRELOAD=libvkblas_hipblas.so python script.py` (reference
 * README.md:60-70).  PyTorch-ROCm bundles its own HIP runtime and loads it
 * under the name libamdhip64.so; a preloaded library that itself depends on
 * libamdhip64.so.7 would pull in the system runtime before PyTorch starts,
 * leaving the process with two HIP runtimes whose streams and handles do not
 * mix.  So the preloaded library (the hipBLAS / rocBLAS / hipBLASLt entry
 * points and these forwarders) has no HIP dependency at all.  The engine is
 * opened at the first GEMM call, when the application has loaded its HIP
 * runtime; the engine's dependency on libamdhip64.so.7 then binds to that
 * runtime by soname (PyTorch's copy carries the same soname), or, in a
 * process without one yet, to the system runtime through the engine's
 * rpath.  The engine is linked -Bsymbolic, so its own calls between these
 * entry points never come back through the forwarders.
 *
 * If the engine cannot be opened, every entry point reports failure
 * (VKBLAS_ERR_INIT; the hipBLAS / rocBLAS / hipBLASLt entry points then
 * forward the call to the vendor library) and the reason is printed once on
 * stderr.  There is no CPU fallback.
 */
#define _GNU_SOURCE
#include <dlfcn.h>
#include <pthread.h>
#include <stdio.h>
#include <string.h>

#include "vkblas_ext.h"

#define ENGINE_NAME "libvkblas_engine.so"

static pthread_once_t g_eng_once = PTHREAD_ONCE_INIT;
static void* g_eng = NULL;

static void stub_anchor(void) {}

static void eng_open(void) {
    Dl_info info;
    char path[4096];
    path[0] = '\0';
    if (dladdr((void*)&stub_anchor, &info) && info.dli_fname) {
        const char* slash = strrchr(info.dli_fname, '/');
        const size_t dir = slash ? (size_t)(slash - info.dli_fname + 1) : 0;
        if (dir + sizeof(ENGINE_NAME) <= sizeof(path)) {
            memcpy(path, info.dli_fname, dir);
            memcpy(path + dir, ENGINE_NAME, sizeof(ENGINE_NAME));
        }
    }
    if (!path[0]) snprintf(path, sizeof(path), "%s", ENGINE_NAME);
    g_eng = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!g_eng) fprintf(stderr, "[vkblas] cannot load the engine %s: %s\n", path, dlerror());
}

static void* eng_sym(const char* name) {
    pthread_once(&g_eng_once, eng_open);
    return g_eng ? dlsym(g_eng, name) : NULL;
}

/* Forwarder: exports `name` with parameter list `params`, calls the engine's
 * `name` with `args`, or returns `err` without an engine. */
#define VKB_ENGINE_FN(ret_t, err, name, params, args)                           \
    ret_t name params {                                                         \
        static void* fn_;                                                       \
        void* f_ = __atomic_load_n(&fn_, __ATOMIC_ACQUIRE);                     \
        if (!f_) {                                                              \
            f_ = eng_sym(#name);                                                \
            __atomic_store_n(&fn_, f_, __ATOMIC_RELEASE);                       \
        }                                                                       \
        return f_ ? ((ret_t(*) params)f_) args : (err);                         \
    }

#define ENGINE_ARGS_F(fp_t)                                                                                      \
    (vkblas_op_t op_a, vkblas_op_t op_b, uint32_t M, uint32_t N, uint32_t K, fp_t alpha, const void* A,          \
     uint32_t lda, const void* B, uint32_t ldb, fp_t beta, void* C, uint32_t ldc, uint32_t batch,                 \
     int64_t stride_a, int64_t stride_b, int64_t stride_c)
#define ENGINE_CALL (op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch, stride_a, stride_b, stride_c)

/* include/vkblas.h */
VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_gemm_f32, ENGINE_ARGS_F(float), ENGINE_CALL)
VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_gemm_f16, ENGINE_ARGS_F(float), ENGINE_CALL)
VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_gemm_bf16, ENGINE_ARGS_F(float), ENGINE_CALL)
VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_gemm_bf16_hipblas, ENGINE_ARGS_F(float), ENGINE_CALL)
VKB_ENGINE_FN(int, VKBLAS_ERR_INIT, vkblas_gemm_f64, ENGINE_ARGS_F(double), ENGINE_CALL)
VKB_ENGINE_FN(int, VKBLAS_ERR_INIT, vkblas_gemm_c64,
              (vkblas_op_t op_a, vkblas_op_t op_b, uint32_t M, uint32_t N, uint32_t K, float alpha_r, float alpha_i,
               const void* A, uint32_t lda, const void* B, uint32_t ldb, float beta_r, float beta_i, void* C,
               uint32_t ldc, uint32_t batch, int64_t stride_a, int64_t stride_b, int64_t stride_c),
              (op_a, op_b, M, N, K, alpha_r, alpha_i, A, lda, B, ldb, beta_r, beta_i, C, ldc, batch, stride_a,
               stride_b, stride_c))
VKB_ENGINE_FN(int, VKBLAS_ERR_INIT, vkblas_gemm_z64,
              (vkblas_op_t op_a, vkblas_op_t op_b, uint32_t M, uint32_t N, uint32_t K, double alpha_r,
               double alpha_i, const void* A, uint32_t lda, const void* B, uint32_t ldb, double beta_r,
               double beta_i, void* C, uint32_t ldc, uint32_t batch, int64_t stride_a, int64_t stride_b,
               int64_t stride_c),
              (op_a, op_b, M, N, K, alpha_r, alpha_i, A, lda, B, ldb, beta_r, beta_i, C, ldc, batch, stride_a,
               stride_b, stride_c))

/* No import cache exists to invalidate (the engine's entry is a no-op too). */
void vkblas_cache_invalidate_base(const void* ptr) { (void)ptr; }

/* include/vkblas_ext.h */
#define ASYNC_PARAMS                                                                                             \
    vkblas_dtype_t ab_type, vkblas_dtype_t c_type, vkblas_op_t op_a, vkblas_op_t op_b, uint32_t M, uint32_t N,    \
        uint32_t K, float alpha, const void* A, uint32_t lda, const void* B, uint32_t ldb, float beta, void* C,  \
        uint32_t ldc, uint32_t batch, int64_t stride_a, int64_t stride_b, int64_t stride_c,                       \
        vkblas_scalar_mode_t scalar_mode, const void* alpha_dev, const void* beta_dev, uint32_t split_k
#define ASYNC_ARGS                                                                                               \
    ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch, stride_a, stride_b,       \
        stride_c, scalar_mode, alpha_dev, beta_dev, split_k

VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_gemm_async, (ASYNC_PARAMS, void* stream),
              (ASYNC_ARGS, stream))
VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_gemm_ex_async,
              (ASYNC_PARAMS, const vkblas_epilogue_t* epilogue, void* stream), (ASYNC_ARGS, epilogue, stream))
VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_gemm_noalloc_async, (ASYNC_PARAMS, void* stream),
              (ASYNC_ARGS, stream))
VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_gemm_batched_async,
              (vkblas_dtype_t ab_type, vkblas_dtype_t c_type, vkblas_op_t op_a, vkblas_op_t op_b, uint32_t M,
               uint32_t N, uint32_t K, float alpha, const void* const* A, uint32_t lda, const void* const* B,
               uint32_t ldb, float beta, void* const* C, uint32_t ldc, uint32_t batch,
               vkblas_scalar_mode_t scalar_mode, const void* alpha_dev, const void* beta_dev, void* stream),
              (ab_type, c_type, op_a, op_b, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc, batch, scalar_mode,
               alpha_dev, beta_dev, stream))
VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_plan_gemm,
              (vkblas_dtype_t ab_type, vkblas_dtype_t c_type, vkblas_op_t op_a, vkblas_op_t op_b, uint32_t M,
               uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb, uint32_t ldc, uint32_t batch, uint32_t split_k,
               int aligned, vkblas_plan_t* plan),
              (ab_type, c_type, op_a, op_b, M, N, K, lda, ldb, ldc, batch, split_k, aligned, plan))
VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_set_override, (int tile, int generic), (tile, generic))
VKB_ENGINE_FN(int, VKBLAS_PATH_NONE, vkblas_last_path, (void), ())
VKB_ENGINE_FN(int, VKBLAS_KERNEL_NONE, vkblas_last_kernel, (void), ())
VKB_ENGINE_FN(size_t, 0, vkblas_noalloc_scratch_bytes, (void), ())
VKB_ENGINE_FN(vkblas_status_t, VKBLAS_ERR_INIT, vkblas_workspace_release, (void), ())
VKB_ENGINE_FN(const char*, "vkblas-mi355x (engine not loaded)", vkblas_version, (void), ())
