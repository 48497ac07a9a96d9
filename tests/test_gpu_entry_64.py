"""The 64-bit-integer (_64) and _v2 forms of the intercepted hipBLAS and
rocBLAS GEMM entry points: hipblasSgemm_64, hipblasHgemm_64, their strided
batched forms, hipblasGemmEx_64 / _v2, hipblasGemmStridedBatchedEx_64 / _v2,
rocblas_gemm_ex_64, rocblas_gemm_strided_batched_ex_64, and the pointer-array
batched hipblasSgemmBatched_64, hipblasHgemmBatched_64,
hipblasGemmBatchedEx_64 and rocblas_gemm_batched_ex_64.  Each call runs
on the same operands as its 32-bit form and must give the same bits (the
same engine call), be computed by this library (a marker call on another
path goes first: a forwarded call would leave the marker's path), and match
the oracle (oracle.ref_gemm_epi_rm on the row-major mapping op_a = transB,
op_b = transA).  The 64-bit forms are hipBLAS 2.x / rocBLAS 4.x additions
the reference did not intercept (src/vkblas_hipblas.c:187-461 covers the
32-bit forms).
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

_vp, _i, _i64, _u32, _ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint32, ctypes.c_longlong
OPN, OPT = 111, 112
HT = {"f32": 0, "f16": 2, "bf16": 14}            # hipDataType
RT = {"f32": 151, "f16": 150, "bf16": 168}       # rocblas_datatype
TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
CONV = {"f32": lambda x: x.astype(np.float32), "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}
BACK = {"f32": lambda x: x.astype(np.float32), "f16": oracle.h2f, "bf16": oracle.bf2f}

SIGS = {
    "hipblasSgemm_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _i64],
    "hipblasHgemm_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _i64],
    "hipblasSgemmStridedBatched_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i64, _ll, _vp, _i64, _ll, _vp, _vp,
                                      _i64, _ll, _i64],
    "hipblasHgemmStridedBatched_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i64, _ll, _vp, _i64, _ll, _vp, _vp,
                                      _i64, _ll, _i64],
    "hipblasGemmEx_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i, _i64, _vp, _i, _i64, _vp, _vp, _i, _i64, _i, _i],
    "hipblasGemmStridedBatchedEx_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i, _i64, _i64, _vp, _i, _i64, _i64,
                                       _vp, _vp, _i, _i64, _i64, _i64, _i, _i],
    "rocblas_gemm_ex": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp, _i, _i, _vp, _vp, _i, _i, _vp, _i, _i, _i, _i,
                        ctypes.c_int32, _u32],
    "rocblas_gemm_ex_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i, _i64, _vp, _i, _i64, _vp, _vp, _i, _i64, _vp, _i,
                           _i64, _i, _i, ctypes.c_int32, _u32],
    "rocblas_gemm_strided_batched_ex": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _i64, _vp, _i, _i, _i64, _vp, _vp, _i,
                                        _i, _i64, _vp, _i, _i, _i64, _i, _i, _i, ctypes.c_int32, _u32],
    "rocblas_gemm_strided_batched_ex_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i, _i64, _i64, _vp, _i, _i64,
                                           _i64, _vp, _vp, _i, _i64, _i64, _vp, _i, _i64, _i64, _i64, _i, _i,
                                           ctypes.c_int32, _u32],
}


class Ctx:
    def __init__(self):
        import vkblas_amd as vk
        from gpu_helpers import Handle
        self.vk = vk
        self.lib = vk.load()
        for name, args in SIGS.items():
            f = getattr(self.lib, name)
            f.argtypes = args
            f.restype = _i
        self.hip = Handle()
        self.hip.set_stream(torch.cuda.current_stream().cuda_stream)
        self.roc_real = ctypes.CDLL("librocblas.so.5")
        self.rh = _vp()
        assert self.roc_real.rocblas_create_handle(ctypes.byref(self.rh)) == 0
        assert self.roc_real.rocblas_set_stream(self.rh, _vp(torch.cuda.current_stream().cuda_stream)) == 0

    def close(self):
        self.hip.close()
        self.roc_real.rocblas_destroy_handle(self.rh)


@pytest.fixture(scope="module")
def ctx():
    c = Ctx()
    yield c
    c.close()


def _marker(vk, path):
    """an engine call on a path other than `path`"""
    x = torch.zeros(65 * 64, dtype=torch.float16, device="cuda:0")
    w = torch.zeros(64 * 64, dtype=torch.float16, device="cuda:0")
    y = torch.zeros(65 * 64, dtype=torch.float16, device="cuda:0")
    rows = 2 if path != vk.PATH_SKINNY else 65
    vk.gemm_async(vk.DT_F16, vk.DT_F16, 0, 1 if rows == 2 else 0, rows, 64, 64, 1.0, x.data_ptr(), 64, w.data_ptr(),
                  64, 0.0, y.data_ptr(), 64)
    torch.cuda.synchronize()
    return vk.last_path()


# (entry, its 32-bit form, A/B type, C type, batch)
ENTRIES = [("hipblasSgemm_64", "hipblasSgemm", "f32", "f32", 1),
           ("hipblasHgemm_64", "hipblasHgemm", "f16", "f16", 1),
           ("hipblasSgemmStridedBatched_64", "hipblasSgemmStridedBatched", "f32", "f32", 3),
           ("hipblasHgemmStridedBatched_64", "hipblasHgemmStridedBatched", "f16", "f16", 3),
           ("hipblasGemmEx_64", "hipblasGemmEx", "bf16", "f32", 1),
           ("hipblasGemmEx_v2", "hipblasGemmEx", "f16", "f32", 1),
           ("hipblasGemmStridedBatchedEx_64", "hipblasGemmStridedBatchedEx", "f16", "f16", 2),
           ("hipblasGemmStridedBatchedEx_v2", "hipblasGemmStridedBatchedEx", "bf16", "bf16", 2),
           ("rocblas_gemm_ex_64", "rocblas_gemm_ex", "f16", "f16", 1),
           ("rocblas_gemm_strided_batched_ex_64", "rocblas_gemm_strided_batched_ex", "bf16", "f32", 2)]


def _call(ctx, name, ab, ct, m, n, k, pa, dA, lda, sa, dB, ldb, sb, pb, dC, ldc, sc, nb):
    lib, h = ctx.lib, ctx.hip.h
    if name in ("hipblasSgemm", "hipblasSgemm_64", "hipblasHgemm", "hipblasHgemm_64"):
        f = getattr(lib, name) if name.endswith("_64") else getattr(ctx.hip.abi, name)
        return f(h, OPT, OPN, m, n, k, pa, dA, lda, dB, ldb, pb, dC, ldc)
    if "gemmStridedBatched" in name and name.startswith("hipblas") and "Ex" not in name:
        f = getattr(lib, name) if name.endswith("_64") else getattr(ctx.hip.abi, name)
        return f(h, OPT, OPN, m, n, k, pa, dA, lda, sa, dB, ldb, sb, pb, dC, ldc, sc, nb)
    if name in ("hipblasGemmEx", "hipblasGemmEx_64", "hipblasGemmEx_v2"):
        f = getattr(lib, name) if name.endswith("_64") else getattr(ctx.hip.abi, name)
        return f(h, OPT, OPN, m, n, k, pa, dA, HT[ab], lda, dB, HT[ab], ldb, pb, dC, HT[ct], ldc, 2, 160)
    if name.startswith("hipblasGemmStridedBatchedEx"):
        f = getattr(lib, name) if name.endswith("_64") else getattr(ctx.hip.abi, name)
        return f(h, OPT, OPN, m, n, k, pa, dA, HT[ab], lda, sa, dB, HT[ab], ldb, sb, pb, dC, HT[ct], ldc, sc, nb,
                 2, 160)
    rh = ctx.rh
    if name.startswith("rocblas_gemm_ex"):
        return getattr(lib, name)(rh, OPT, OPN, m, n, k, pa, dA, RT[ab], lda, dB, RT[ab], ldb, pb, dC, RT[ct], ldc,
                                  dC, RT[ct], ldc, 151, 0, 0, 0)
    return getattr(lib, name)(rh, OPT, OPN, m, n, k, pa, dA, RT[ab], lda, sa, dB, RT[ab], ldb, sb, pb, dC, RT[ct],
                              ldc, sc, dC, RT[ct], ldc, sc, nb, 151, 0, 0, 0)


@pytest.mark.parametrize("entry", ENTRIES, ids=lambda e: e[0])
def test_64_and_v2_forms_match_32_bit_forms(ctx, entry):
    from gpu_helpers import normwise, f32_bound, F16_BOUND, BF16_BOUND
    vk = ctx.vk
    name, base, ab, ct, nb = entry
    print(f"[case] entry {name} against {base}", flush=True)
    m, n, k = 264, 136, 200                 # A stored k x m (transA = T), B k x n
    lda, ldb, ldc = k + 8, k + 16, m + 8
    sa, sb, sc = m * lda + 64, n * ldb + 64, n * ldc + 64
    r = np.random.default_rng(sum(map(ord, name)))
    A = CONV[ab]((r.standard_normal(sa * nb) * 0.5).astype(np.float32))
    B = CONV[ab]((r.standard_normal(sb * nb) * 0.05).astype(np.float32))
    C = CONV[ct](r.standard_normal(sc * nb).astype(np.float32))

    def dev(x, t):
        return torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x).view(TD[t]).to("cuda:0")
    dA, dB = dev(A, ab), dev(B, ab)
    alpha, beta = 1.25, -0.5
    half = name.startswith("hipblasH")
    if half:
        sa_, sb_ = [ctypes.c_uint16(int(np.array([v], np.float16).view(np.uint16)[0])) for v in (alpha, beta)]
    else:
        sa_, sb_ = ctypes.c_float(alpha), ctypes.c_float(beta)
    dt = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    pl = vk.plan(dt[ab], dt[ct], 0, 1, n, m, k, ldb, lda, ldc, nb)
    outs = []
    for fn in (base, name):
        dC = dev(C, ct)
        marker = _marker(vk, pl.path)
        st = _call(ctx, fn, ab, ct, m, n, k, ctypes.byref(sa_), dA.data_ptr(), lda, sa, dB.data_ptr(), ldb, sb,
                   ctypes.byref(sb_), dC.data_ptr(), ldc, sc, nb)
        torch.cuda.synchronize()
        assert st == 0, (fn, st)
        assert vk.last_path() == pl.path != marker, f"{fn} was forwarded"
        got = dC.cpu()
        outs.append(got.view(torch.int16).numpy().view(np.uint16) if ct != "f32" else got.numpy())
    assert np.array_equal(outs[0].view(np.uint8), outs[1].view(np.uint8)), f"{name} differs from {base}"
    bound = f32_bound(k) if (ab, ct) == ("f32", "f32") else (BF16_BOUND if ct == "bf16" else F16_BOUND)
    for b in range(nb):
        want = C[b * sc:(b + 1) * sc].copy()
        # column-major C(m x n) = row-major C'(n x m) = op(B)' op(A)': op_a = N (B: n rows of k), op_b = T (A)
        oracle.ref_gemm_epi_rm(ab, ct, 0, 1, n, m, k, np.ascontiguousarray(B[b * sb:(b + 1) * sb]), ldb,
                               np.ascontiguousarray(A[b * sa:(b + 1) * sa]), lda, alpha, beta, want.copy(), ldc, want,
                               ldc, None)
        g = BACK[ct](outs[1][b * sc:(b + 1) * sc][: n * ldc].reshape(n, ldc)[:, :m])
        w = BACK[ct](want[: n * ldc].reshape(n, ldc)[:, :m])
        assert normwise(g, w) <= bound, b


# Pointer-array batched forms: hipblasSgemmBatched_64, hipblasHgemmBatched_64,
# hipblasGemmBatchedEx_64 and rocblas_gemm_batched_ex_64 against their 32-bit
# forms (themselves checked against the oracle in test_gpu_batched_ptr.py and
# test_gpu_rocblas.py), bitwise, each computed here.
PSIGS = {
    "hipblasSgemmBatched_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64],
    "hipblasHgemmBatched_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _i64, _i64],
    "hipblasGemmBatchedEx_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i, _i64, _vp, _i, _i64, _vp, _vp, _i, _i64,
                                _i64, _i, _i],
    "rocblas_gemm_batched_ex": [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp, _i, _i, _vp, _vp, _i, _i, _vp, _i, _i,
                                _i, _i, _i, ctypes.c_int32, _u32],
    "rocblas_gemm_batched_ex_64": [_vp, _i, _i, _i64, _i64, _i64, _vp, _vp, _i, _i64, _vp, _i, _i64, _vp, _vp, _i,
                                   _i64, _vp, _i, _i64, _i64, _i, _i, ctypes.c_int32, _u32],
}
PENTRIES = [("hipblasSgemmBatched_64", "hipblasSgemmBatched", "f32", "f32"),
            ("hipblasHgemmBatched_64", "hipblasHgemmBatched", "f16", "f16"),
            ("hipblasGemmBatchedEx_64", "hipblasGemmBatchedEx", "bf16", "f32"),
            ("rocblas_gemm_batched_ex_64", "rocblas_gemm_batched_ex", "f16", "f16")]


@pytest.mark.parametrize("entry", PENTRIES, ids=lambda e: e[0])
def test_64_pointer_array_forms_match_32_bit_forms(ctx, entry):
    vk = ctx.vk
    for nm, args in PSIGS.items():
        f = getattr(ctx.lib, nm)
        f.argtypes = args
        f.restype = _i
    name, base, ab, ct = entry
    print(f"[case] pointer-array entry {name} against {base}", flush=True)
    m, n, k, nb = 200, 72, 136, 3
    lda, ldb, ldc = k + 8, k, m + 8                   # A stored k x m (transA = T), B k x n (N)
    r = np.random.default_rng(sum(map(ord, name)))

    def dev(x, t):
        return torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x).view(TD[t]).to("cuda:0")
    As = [dev(CONV[ab]((r.standard_normal(m * lda) * 0.5).astype(np.float32)), ab) for _ in range(nb)]
    Bs = [dev(CONV[ab]((r.standard_normal(n * ldb) * 0.05).astype(np.float32)), ab) for _ in range(nb)]
    C0 = [CONV[ct](r.standard_normal(n * ldc).astype(np.float32)) for _ in range(nb)]
    pA = torch.tensor([t.data_ptr() for t in As], dtype=torch.int64, device="cuda:0")
    pB = torch.tensor([t.data_ptr() for t in Bs], dtype=torch.int64, device="cuda:0")
    alpha, beta = 0.75, 0.5
    half = name.startswith("hipblasH")
    if half:
        sa_, sb_ = [ctypes.c_uint16(int(np.array([v], np.float16).view(np.uint16)[0])) for v in (alpha, beta)]
    else:
        sa_, sb_ = ctypes.c_float(alpha), ctypes.c_float(beta)
    outs = []
    for fn in (base, name):
        Cs = [dev(c, ct) for c in C0]
        pC = torch.tensor([t.data_ptr() for t in Cs], dtype=torch.int64, device="cuda:0")
        marker = _marker(vk, vk.PATH_TILE64)        # pointer arrays run the checked 64x64 kernel
        h = ctx.hip.h
        if fn in ("hipblasSgemmBatched", "hipblasHgemmBatched"):
            st = getattr(ctx.hip.abi, fn)(h, OPT, OPN, m, n, k, ctypes.byref(sa_), pA.data_ptr(), lda,
                                          pB.data_ptr(), ldb, ctypes.byref(sb_), pC.data_ptr(), ldc, nb)
        elif fn in ("hipblasSgemmBatched_64", "hipblasHgemmBatched_64"):
            st = getattr(ctx.lib, fn)(h, OPT, OPN, m, n, k, ctypes.byref(sa_), pA.data_ptr(), lda, pB.data_ptr(), ldb,
                                      ctypes.byref(sb_), pC.data_ptr(), ldc, nb)
        elif fn == "hipblasGemmBatchedEx":
            st = ctx.hip.abi.hipblasGemmBatchedEx(h, OPT, OPN, m, n, k, ctypes.byref(sa_), pA.data_ptr(), HT[ab], lda,
                                                  pB.data_ptr(), HT[ab], ldb, ctypes.byref(sb_), pC.data_ptr(),
                                                  HT[ct], ldc, nb, 2, 160)
        elif fn == "hipblasGemmBatchedEx_64":
            st = ctx.lib.hipblasGemmBatchedEx_64(h, OPT, OPN, m, n, k, ctypes.byref(sa_), pA.data_ptr(), HT[ab], lda,
                                                 pB.data_ptr(), HT[ab], ldb, ctypes.byref(sb_), pC.data_ptr(), HT[ct],
                                                 ldc, nb, 2, 160)
        else:
            st = getattr(ctx.lib, fn)(ctx.rh, OPT, OPN, m, n, k, ctypes.byref(sa_), pA.data_ptr(), RT[ab], lda,
                                      pB.data_ptr(), RT[ab], ldb, ctypes.byref(sb_), pC.data_ptr(), RT[ct], ldc,
                                      pC.data_ptr(), RT[ct], ldc, nb, 151, 0, 0, 0)
        torch.cuda.synchronize()
        assert st == 0, (fn, st)
        # the marker left PATH_SKINNY: a forwarded call would not replace it
        assert marker == vk.PATH_SKINNY
        assert vk.last_path() == vk.PATH_TILE64 and vk.last_kernel() == vk.KERNEL_GENERIC_CHECKED, (fn, vk.last_path())
        outs.append([c.cpu().view(torch.int16 if ct != "f32" else torch.int32).numpy().copy() for c in Cs])
    for b in range(nb):
        assert np.array_equal(outs[0][b], outs[1][b]), f"{name} differs from {base}, batch {b}"
