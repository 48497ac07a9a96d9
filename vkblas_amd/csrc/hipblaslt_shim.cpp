// hipblaslt_shim.cpp — hipBLASLt entry points of libvkblas_hipblas.so (host
// C++17, no device code).
//
// PyTorch-ROCm on gfx950 sends mm / bmm / addmm / linear to hipblasLtMatmul;
// interposing it makes the reference's plain `LD_PRELOAD=libvkblas_hipblas.so
// python script.py` usage (reference README.md:60-70) reach this library's
// kernels, as the reference reached its engine by interposing the layer
// PyTorch called (src/vkblas_hipblas.c:802-808).
//
// hipblasLtMatmul is column-major: D(m x n) = alpha op(A) op(B) + beta C
// (+ bias[row] with HIPBLASLT_EPILOGUE_BIAS).  As at the hipBLAS layer
// (reference src/vkblas_hipblas.c:187-189) it is the row-major
// D'(n x m) = op(B)' op(A)', so the engine runs with
//     op_a = transB, op_b = transA, M = n, N = m, A = B, B = A,
// C as the separate C input, and the bias on the engine's columns.
//
// What a matmul descriptor and a matrix layout hold cannot be read back
// through the hipBLASLt API in general (PyTorch's bundled hipBLASLt answers
// only a layout's batch count and stride, and nothing gives a descriptor's
// compute and scale types), so the calls that create, change and destroy
// them are interposed too: each is forwarded unchanged to the real library
// and, when it succeeds, recorded here.  A matmul is computed only when
// everything its descriptor and layouts were given is recorded and
// supported; anything else (an object created before this library was
// loaded, scale pointers, activation or gradient epilogues, other orders,
// fp8 ...) is forwarded to the real hipblasLtMatmul untouched.
#include <dlfcn.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "vkblas_ext.h"
#include "vkblas_hipblaslt.h"

namespace {

// ------------------------------------------------------ real hipBLASLt lookup

pthread_once_t g_once = PTHREAD_ONCE_INIT;
void* g_real = nullptr;
void* g_self_base = nullptr;
int g_trace = 0;

void self_anchor() {}

bool in_self(void* f) {
    Dl_info info;
    if (!f || !dladdr(f, &info)) return false;
    return info.dli_fbase == g_self_base;
}

void real_open() {
    Dl_info info;
    const char* e = getenv("VKBLAS_TRACE");
    g_trace = e && e[0] && e[0] != '0';
    if (dladdr((void*)&self_anchor, &info)) g_self_base = info.dli_fbase;
    static const char* names[] = {"libhipblaslt.so.1", "libhipblaslt.so", "/opt/rocm/lib/libhipblaslt.so.1"};
    // prefer the instance the process already uses (its handles, descriptors
    // and layouts are that instance's objects)
    for (int pass = 0; pass < 2 && !g_real; ++pass) {
        for (const char* n : names) {
            void* h = dlopen(n, RTLD_LAZY | (pass == 0 ? RTLD_NOLOAD : RTLD_LOCAL));
            if (!h) continue;
            void* probe = dlsym(h, "hipblasLtMatmul");
            if (probe && !in_self(probe)) {
                g_real = h;
                break;
            }
            dlclose(h);
        }
    }
    if (!g_real && g_trace) fprintf(stderr, "[vkblas] real libhipblaslt not found: forwarding disabled\n");
}

// A symbol of the real hipBLASLt, never one of ours.
void* real_sym(const char* name) {
    pthread_once(&g_once, real_open);
    void* f = dlsym(RTLD_NEXT, name);
    if (f && !in_self(f)) return f;
    if (g_real) {
        f = dlsym(g_real, name);
        if (f && !in_self(f)) return f;
    }
    return nullptr;
}

template <typename Fn>
Fn cached(void** slot, const char* name) {
    void* f = __atomic_load_n(slot, __ATOMIC_ACQUIRE);
    if (!f) {
        f = real_sym(name);
        __atomic_store_n(slot, f, __ATOMIC_RELEASE);
    }
    return (Fn)f;
}

// ---------------------------------------------------------------- records

// What a descriptor was created and set with.  `foreign` marks anything set
// that this library does not compute (scale pointers, amax, scaling modes,
// attributes it does not know).
struct DescRec {
    int compute = 0, scale = 0;
    int32_t ta = HIPBLAS_OP_N, tb = HIPBLAS_OP_N;
    uint32_t epilogue = HIPBLASLT_EPILOGUE_DEFAULT;
    const void* bias = nullptr;
    int32_t bias_type = (int32_t)HIPBLASLT_DATATYPE_INVALID;
    int32_t pmode = HIPBLASLT_POINTER_MODE_HOST;
    bool foreign = false;
};

struct LayRec {
    uint32_t type = 0;
    uint64_t rows = 0, cols = 0;
    int64_t ld = 0;
    int32_t order = HIPBLASLT_ORDER_COL;
    int32_t batch = 1;
    int64_t stride = 0;
    bool foreign = false;
};

// Open addressing on the object's address, linear probing, backward-shift
// deletion, one lock.  An object that finds the table full is not recorded
// (its matmuls are forwarded).
template <typename Rec>
class Table {
  public:
    void put(const void* key, const Rec& r) {
        Lock l(this);
        unsigned i = home(key);
        for (int probe = 0; probe < kSlots; ++probe, i = (i + 1) & kMask) {
            if (!slot_[i].key || slot_[i].key == key) {
                slot_[i].key = key;
                slot_[i].rec = r;
                return;
            }
        }
    }
    // a copy of the record, or false
    bool get(const void* key, Rec* out) {
        Lock l(this);
        const int i = find(key);
        if (i < 0) return false;
        *out = slot_[i].rec;
        return true;
    }
    template <typename F>
    void update(const void* key, F&& f) {
        Lock l(this);
        const int i = find(key);
        if (i >= 0) f(slot_[i].rec);
    }
    void erase(const void* key) {
        Lock l(this);
        const int i = find(key);
        if (i < 0) return;
        unsigned hole = (unsigned)i, j = (hole + 1) & kMask;
        while (slot_[j].key) {
            // move j back into the hole unless its home lies in (hole, j]
            if (((j - home(slot_[j].key)) & kMask) >= ((j - hole) & kMask)) {
                slot_[hole] = slot_[j];
                hole = j;
            }
            j = (j + 1) & kMask;
        }
        slot_[hole].key = nullptr;
    }

  private:
    static constexpr int kSlots = 4096;
    static constexpr unsigned kMask = kSlots - 1;
    struct Slot {
        const void* key = nullptr;
        Rec rec;
    };
    struct Lock {
        explicit Lock(Table* t) : t_(t) { pthread_mutex_lock(&t_->mu_); }
        ~Lock() { pthread_mutex_unlock(&t_->mu_); }
        Table* t_;
    };
    static unsigned home(const void* key) {
        uint64_t x = (uint64_t)(uintptr_t)key;
        x ^= x >> 33;
        x *= 0xff51afd7ed558ccdull;
        x ^= x >> 33;
        return (unsigned)(x & kMask);
    }
    int find(const void* key) const {
        unsigned i = home(key);
        for (int probe = 0; probe < kSlots && slot_[i].key; ++probe, i = (i + 1) & kMask)
            if (slot_[i].key == key) return (int)i;
        return -1;
    }
    Slot slot_[kSlots];
    pthread_mutex_t mu_ = PTHREAD_MUTEX_INITIALIZER;
};

Table<DescRec> g_descs;
Table<LayRec> g_lays;

template <typename V>
bool read_value(const void* buf, size_t size, V* out) {
    if (!buf || size != sizeof(V)) return false;
    memcpy(out, buf, sizeof(V));
    return true;
}

bool all_zero(const void* buf, size_t size) {
    const unsigned char* p = (const unsigned char*)buf;
    for (size_t i = 0; buf && i < size; ++i)
        if (p[i]) return false;
    return true;
}

void record_desc_attr(DescRec& r, int attr, const void* buf, size_t size) {
    bool ok = true;
    switch (attr) {
        case HIPBLASLT_MATMUL_DESC_TRANSA: ok = read_value(buf, size, &r.ta); break;
        case HIPBLASLT_MATMUL_DESC_TRANSB: ok = read_value(buf, size, &r.tb); break;
        case HIPBLASLT_MATMUL_DESC_EPILOGUE: ok = read_value(buf, size, &r.epilogue); break;
        case HIPBLASLT_MATMUL_DESC_BIAS_POINTER: ok = read_value(buf, size, &r.bias); break;
        case HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE: ok = read_value(buf, size, &r.bias_type); break;
        case HIPBLASLT_MATMUL_DESC_POINTER_MODE: ok = read_value(buf, size, &r.pmode); break;
        // only an activation epilogue or an fp8 / mixed compute reads these;
        // full fp32 arithmetic satisfies any compute-input type request
        case HIPBLASLT_MATMUL_DESC_EPILOGUE_AUX_POINTER:
        case HIPBLASLT_MATMUL_DESC_EPILOGUE_AUX_LD:
        case HIPBLASLT_MATMUL_DESC_EPILOGUE_AUX_BATCH_STRIDE:
        case HIPBLASLT_MATMUL_DESC_EPILOGUE_AUX_DATA_TYPE:
        case HIPBLASLT_MATMUL_DESC_COMPUTE_INPUT_TYPE_A_EXT:
        case HIPBLASLT_MATMUL_DESC_COMPUTE_INPUT_TYPE_B_EXT:
        case HIPBLASLT_MATMUL_DESC_EPILOGUE_ACT_ARG0_EXT:
        case HIPBLASLT_MATMUL_DESC_EPILOGUE_ACT_ARG1_EXT:
            break;
        // scaling pointers and modes, amax, anything unknown: only their
        // defaults (all zero) are computed here
        default: ok = all_zero(buf, size); break;
    }
    if (!ok) r.foreign = true;
}

void record_layout_attr(LayRec& r, int attr, const void* buf, size_t size) {
    bool ok = true;
    switch (attr) {
        case HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT: ok = read_value(buf, size, &r.batch); break;
        case HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET: ok = read_value(buf, size, &r.stride); break;
        case HIPBLASLT_MATRIX_LAYOUT_TYPE: ok = read_value(buf, size, &r.type); break;
        case HIPBLASLT_MATRIX_LAYOUT_ORDER: ok = read_value(buf, size, &r.order); break;
        case HIPBLASLT_MATRIX_LAYOUT_ROWS: ok = read_value(buf, size, &r.rows); break;
        case HIPBLASLT_MATRIX_LAYOUT_COLS: ok = read_value(buf, size, &r.cols); break;
        case HIPBLASLT_MATRIX_LAYOUT_LD: ok = read_value(buf, size, &r.ld); break;
        default: ok = false; break;
    }
    if (!ok) r.foreign = true;
}

// ----------------------------------------------------------------- matmul

bool dtype_of(uint32_t t, vkblas_dtype_t* out) {
    if (t == HIP_R_32F) { *out = VKBLAS_DT_F32; return true; }
    if (t == HIP_R_16F) { *out = VKBLAS_DT_F16; return true; }
    if (t == HIP_R_16BF) { *out = VKBLAS_DT_BF16; return true; }
    return false;
}

const char* tname(vkblas_dtype_t t) { return t == VKBLAS_DT_F16 ? "f16" : t == VKBLAS_DT_BF16 ? "bf16" : "f32"; }

bool compute_f32(int c) {
    return c == HIPBLAS_COMPUTE_32F || c == HIPBLAS_COMPUTE_32F_PEDANTIC || c == HIPBLAS_COMPUTE_32F_FAST_16F ||
           c == HIPBLAS_COMPUTE_32F_FAST_16BF || c == HIPBLAS_COMPUTE_32F_FAST_TF32;
}

bool op_t(int32_t op) { return op == HIPBLAS_OP_T || op == HIPBLAS_OP_C; }

// false, with the reason on stderr under VKBLAS_TRACE: the caller forwards
bool decline(const char* why) {
    if (g_trace) fprintf(stderr, "[vkblas] hipblaslt matmul forwarded: %s\n", why);
    return false;
}

bool run(hipblasLtMatmulDesc_t desc, const void* alpha, const void* A, hipblasLtMatrixLayout_t Adesc,
         const void* B, hipblasLtMatrixLayout_t Bdesc, const void* beta, const void* C,
         hipblasLtMatrixLayout_t Cdesc, void* D, hipblasLtMatrixLayout_t Ddesc, hipStream_t stream,
         bool* failed) {
    // *failed: the engine failed after part of D was written (not forwarded)
    *failed = false;
    pthread_once(&g_once, real_open);
    if (!desc || !alpha || !beta || !A || !B || !D) return decline("null argument");
    DescRec dr;
    if (!g_descs.get(desc, &dr)) return decline("descriptor not created through this library");
    if (dr.foreign) return decline("descriptor attribute not computed here (scale / amax / unknown)");
    if (!compute_f32(dr.compute) || dr.scale != HIP_R_32F) return decline("compute or scale type");
    if (dr.epilogue != HIPBLASLT_EPILOGUE_DEFAULT && dr.epilogue != HIPBLASLT_EPILOGUE_BIAS)
        return decline("epilogue");
    if (dr.pmode != HIPBLASLT_POINTER_MODE_HOST && dr.pmode != HIPBLASLT_POINTER_MODE_DEVICE)
        return decline("pointer mode");

    LayRec la, lb, lc, ld;
    if (!g_lays.get(Adesc, &la) || !g_lays.get(Bdesc, &lb) || !g_lays.get(Ddesc, &ld))
        return decline("layout not created through this library");
    const bool have_c = Cdesc != nullptr && C != nullptr;
    if (have_c && !g_lays.get(Cdesc, &lc)) return decline("layout not created through this library");
    if (la.foreign || lb.foreign || ld.foreign || (have_c && lc.foreign)) return decline("layout attribute");
    if (la.order != HIPBLASLT_ORDER_COL || lb.order != HIPBLASLT_ORDER_COL || ld.order != HIPBLASLT_ORDER_COL ||
        (have_c && lc.order != HIPBLASLT_ORDER_COL))
        return decline("order");
    vkblas_dtype_t at, bt, ct, dt;
    if (!dtype_of(la.type, &at) || !dtype_of(lb.type, &bt) || !dtype_of(ld.type, &dt) || at != bt)
        return decline("data types");
    if (have_c && (!dtype_of(lc.type, &ct) || ct != dt)) return decline("C type");

    // column-major shapes: D m x n, op(A) m x k, op(B) k x n
    const uint64_t m = ld.rows, n = ld.cols;
    const uint64_t k = op_t(dr.ta) ? la.rows : la.cols;
    if ((op_t(dr.ta) ? la.cols : la.rows) != m || (op_t(dr.tb) ? lb.cols : lb.rows) != k ||
        (op_t(dr.tb) ? lb.rows : lb.cols) != n || (have_c && (lc.rows != m || lc.cols != n)))
        return decline("shapes disagree");
    const int32_t batch = ld.batch;
    if (batch < 1 || la.batch != batch || lb.batch != batch || (have_c && lc.batch != batch))
        return decline("batch counts");
    if (m == 0 || n == 0 || k == 0 || m > UINT32_MAX || n > UINT32_MAX || k > UINT32_MAX) return decline("sizes");
    if (la.ld < (int64_t)la.rows || lb.ld < (int64_t)lb.rows || ld.ld < (int64_t)m ||
        (have_c && lc.ld < (int64_t)m) || la.ld > UINT32_MAX || lb.ld > UINT32_MAX || ld.ld > UINT32_MAX ||
        (have_c && lc.ld > UINT32_MAX))
        return decline("leading dimensions");

    vkblas_epilogue_t epi;
    memset(&epi, 0, sizeof(epi));
    if (dr.epilogue == HIPBLASLT_EPILOGUE_BIAS) {
        if (!dr.bias) return decline("bias epilogue without a bias");
        vkblas_dtype_t bdt = dt;   // unset: the type of D
        if (dr.bias_type != (int32_t)HIPBLASLT_DATATYPE_INVALID && !dtype_of((uint32_t)dr.bias_type, &bdt))
            return decline("bias type");
        epi.bias = dr.bias;
        epi.bias_type = bdt;
    }

    float a = 0.0f, b = 0.0f;
    vkblas_scalar_mode_t sm = VKBLAS_SCALAR_HOST;
    const void* ad = nullptr;
    const void* bd = nullptr;
    bool beta_zero = false;
    if (dr.pmode == HIPBLASLT_POINTER_MODE_DEVICE) {
        sm = VKBLAS_SCALAR_DEV_F32;
        ad = alpha;
        bd = beta;
    } else {
        a = *(const float*)alpha;
        b = *(const float*)beta;
        beta_zero = b == 0.0f;
    }
    // beta's matrix: C when it is not D (C == D is the in-place form)
    if (have_c && C == D && (lc.ld != ld.ld || (batch > 1 && lc.stride != ld.stride)))
        return decline("C aliases D with another layout");
    if (have_c && C != D) {
        epi.c_in = C;
        epi.ldc_in = (uint32_t)lc.ld;
        epi.stride_c_in = lc.stride;
    } else if (!have_c && !beta_zero) {
        return decline("beta may be nonzero without C");
    }
    if (g_trace)
        fprintf(stderr, "[vkblas] hipblaslt matmul %s%s %s->%s m=%llu n=%llu k=%llu lda=%lld ldb=%lld ldd=%lld "
                        "batch=%d%s%s\n",
                op_t(dr.ta) ? "T" : "N", op_t(dr.tb) ? "T" : "N", tname(at), tname(dt), (unsigned long long)m,
                (unsigned long long)n, (unsigned long long)k, (long long)la.ld, (long long)lb.ld, (long long)ld.ld,
                batch, epi.bias ? " bias" : "", epi.c_in ? " c!=d" : "");
    const vkblas_op_t op_a = op_t(dr.tb) ? VKBLAS_OP_T : VKBLAS_OP_N;
    const vkblas_op_t op_b = op_t(dr.ta) ? VKBLAS_OP_T : VKBLAS_OP_N;
    const vkblas_status_t st = vkblas_gemm_ex_async(
        at, dt, op_a, op_b, (uint32_t)n, (uint32_t)m, (uint32_t)k, a, B, (uint32_t)lb.ld, A, (uint32_t)la.ld, b, D,
        (uint32_t)ld.ld, (uint32_t)batch, batch > 1 ? lb.stride : 0, batch > 1 ? la.stride : 0,
        batch > 1 ? ld.stride : 0, sm, ad, bd, 0, (epi.bias || epi.c_in) ? &epi : nullptr, (void*)stream);
    if (st == VKBLAS_ERR_PARTIAL) {
        if (g_trace) fprintf(stderr, "[vkblas] engine status %d: execution failed, not forwarded\n", (int)st);
        *failed = true;
        return false;
    }
    if (st != VKBLAS_OK) {
        if (g_trace) fprintf(stderr, "[vkblas] engine status %d: forwarding\n", (int)st);
        return false;
    }
    return true;
}

void* g_desc_create_fn;
void* g_desc_destroy_fn;
void* g_desc_set_fn;
void* g_lay_create_fn;
void* g_lay_destroy_fn;
void* g_lay_set_fn;
void* g_matmul_fn;

}  // namespace

extern "C" {

hipblasStatus_t hipblasLtMatmulDescCreate(hipblasLtMatmulDesc_t* matmulDesc, hipblasComputeType_t computeType,
                                          hipDataType scaleType) {
    typedef hipblasStatus_t (*fn_t)(hipblasLtMatmulDesc_t*, hipblasComputeType_t, hipDataType);
    fn_t f = cached<fn_t>(&g_desc_create_fn, "hipblasLtMatmulDescCreate");
    if (!f) return HIPBLAS_STATUS_NOT_INITIALIZED;
    const hipblasStatus_t st = f(matmulDesc, computeType, scaleType);
    if (st == HIPBLAS_STATUS_SUCCESS && matmulDesc && *matmulDesc) {
        DescRec r;
        r.compute = (int)computeType;
        r.scale = (int)scaleType;
        g_descs.put(*matmulDesc, r);
    }
    return st;
}

hipblasStatus_t hipblasLtMatmulDescDestroy(const hipblasLtMatmulDesc_t matmulDesc) {
    typedef hipblasStatus_t (*fn_t)(const hipblasLtMatmulDesc_t);
    if (matmulDesc) g_descs.erase(matmulDesc);
    fn_t f = cached<fn_t>(&g_desc_destroy_fn, "hipblasLtMatmulDescDestroy");
    return f ? f(matmulDesc) : HIPBLAS_STATUS_NOT_INITIALIZED;
}

hipblasStatus_t hipblasLtMatmulDescSetAttribute(hipblasLtMatmulDesc_t matmulDesc,
                                                hipblasLtMatmulDescAttributes_t attr, const void* buf,
                                                size_t sizeInBytes) {
    typedef hipblasStatus_t (*fn_t)(hipblasLtMatmulDesc_t, hipblasLtMatmulDescAttributes_t, const void*, size_t);
    fn_t f = cached<fn_t>(&g_desc_set_fn, "hipblasLtMatmulDescSetAttribute");
    if (!f) return HIPBLAS_STATUS_NOT_INITIALIZED;
    const hipblasStatus_t st = f(matmulDesc, attr, buf, sizeInBytes);
    if (st == HIPBLAS_STATUS_SUCCESS && matmulDesc)
        g_descs.update(matmulDesc, [&](DescRec& r) { record_desc_attr(r, (int)attr, buf, sizeInBytes); });
    return st;
}

hipblasStatus_t hipblasLtMatrixLayoutCreate(hipblasLtMatrixLayout_t* matLayout, hipDataType type, uint64_t rows,
                                            uint64_t cols, int64_t ld) {
    typedef hipblasStatus_t (*fn_t)(hipblasLtMatrixLayout_t*, hipDataType, uint64_t, uint64_t, int64_t);
    fn_t f = cached<fn_t>(&g_lay_create_fn, "hipblasLtMatrixLayoutCreate");
    if (!f) return HIPBLAS_STATUS_NOT_INITIALIZED;
    const hipblasStatus_t st = f(matLayout, type, rows, cols, ld);
    if (st == HIPBLAS_STATUS_SUCCESS && matLayout && *matLayout) {
        LayRec r;
        r.type = (uint32_t)type;
        r.rows = rows;
        r.cols = cols;
        r.ld = ld;
        g_lays.put(*matLayout, r);
    }
    return st;
}

hipblasStatus_t hipblasLtMatrixLayoutDestroy(const hipblasLtMatrixLayout_t matLayout) {
    typedef hipblasStatus_t (*fn_t)(const hipblasLtMatrixLayout_t);
    if (matLayout) g_lays.erase(matLayout);
    fn_t f = cached<fn_t>(&g_lay_destroy_fn, "hipblasLtMatrixLayoutDestroy");
    return f ? f(matLayout) : HIPBLAS_STATUS_NOT_INITIALIZED;
}

hipblasStatus_t hipblasLtMatrixLayoutSetAttribute(hipblasLtMatrixLayout_t matLayout,
                                                  hipblasLtMatrixLayoutAttribute_t attr, const void* buf,
                                                  size_t sizeInBytes) {
    typedef hipblasStatus_t (*fn_t)(hipblasLtMatrixLayout_t, hipblasLtMatrixLayoutAttribute_t, const void*, size_t);
    fn_t f = cached<fn_t>(&g_lay_set_fn, "hipblasLtMatrixLayoutSetAttribute");
    if (!f) return HIPBLAS_STATUS_NOT_INITIALIZED;
    const hipblasStatus_t st = f(matLayout, attr, buf, sizeInBytes);
    if (st == HIPBLAS_STATUS_SUCCESS && matLayout)
        g_lays.update(matLayout, [&](LayRec& r) { record_layout_attr(r, (int)attr, buf, sizeInBytes); });
    return st;
}

hipblasStatus_t hipblasLtMatmul(hipblasLtHandle_t handle, hipblasLtMatmulDesc_t matmulDesc, const void* alpha,
                                const void* A, hipblasLtMatrixLayout_t Adesc, const void* B,
                                hipblasLtMatrixLayout_t Bdesc, const void* beta, const void* C,
                                hipblasLtMatrixLayout_t Cdesc, void* D, hipblasLtMatrixLayout_t Ddesc,
                                const hipblasLtMatmulAlgo_t* algo, void* workspace, size_t workspaceSizeInBytes,
                                hipStream_t stream) {
    bool failed = false;
    if (handle && run(matmulDesc, alpha, A, Adesc, B, Bdesc, beta, C, Cdesc, D, Ddesc, stream, &failed))
        return HIPBLAS_STATUS_SUCCESS;
    if (failed) return HIPBLAS_STATUS_EXECUTION_FAILED;
    typedef hipblasStatus_t (*fn_t)(hipblasLtHandle_t, hipblasLtMatmulDesc_t, const void*, const void*,
                                    hipblasLtMatrixLayout_t, const void*, hipblasLtMatrixLayout_t, const void*,
                                    const void*, hipblasLtMatrixLayout_t, void*, hipblasLtMatrixLayout_t,
                                    const hipblasLtMatmulAlgo_t*, void*, size_t, hipStream_t);
    fn_t f = cached<fn_t>(&g_matmul_fn, "hipblasLtMatmul");
    return f ? f(handle, matmulDesc, alpha, A, Adesc, B, Bdesc, beta, C, Cdesc, D, Ddesc, algo, workspace,
                 workspaceSizeInBytes, stream)
             : HIPBLAS_STATUS_NOT_INITIALIZED;
}

}  // extern "C"
