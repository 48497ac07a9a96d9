"""Seeded random sweep through the hipBLAS entry points of the drop-in
library (the boundary PyTorch and the reference's tests call: column-major
hipblasSgemm / Hgemm / GemmEx and their strided-batched forms,
src/vkblas_hipblas.c:826-844 for the reference's operand swap), every result
checked against the oracle and every call asserted computed by the engine
(not forwarded to the vendor library).

Each case draws the entry point, the GemmEx type triple (compute 32F), the
three transposes (N, T and C, which is T for real data), m / n / k from a
shape class, leading dimensions at or above the hipBLAS minimum with NaN in
the padding, alpha and beta (beta == 0 over a C full of NaN), host or
device pointer mode and, for the strided forms, a batch of 2-3 with gaps of
NaN between the matrices.  The oracle sees the engine's row-major form of
the call: hipBLAS C (m x n, column-major) is the engine's n x m row-major
C = op(B)' op(A)', so op_a = transB, op_b = transA.  Bars as in the other
GPU tests (normwise: fp32 1e-5 sqrt(k), fp16 and 16-bit -> fp32 2e-3, bf16
8e-3), large outputs on 16 sampled rows.
"""
import ctypes

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

NCASES = 200
# (A/B type, C type) of GemmEx with compute 32F
EX = [("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32"), ("f32", "f32"), ("f32", "f16"),
      ("f32", "bf16")]
NAN = {"f32": np.float32(np.nan), "f16": np.uint16(0x7E00), "bf16": np.uint16(0x7FC0)}
CONV = {"f32": lambda x: x.astype(np.float32), "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}
BACK = {"f32": lambda x: x.astype(np.float32), "f16": oracle.h2f, "bf16": oracle.bf2f}


def _draw(i):
    r = np.random.default_rng(7000 + i)
    entry = str(r.choice(["Sgemm", "Hgemm", "GemmEx", "SgemmStridedBatched", "HgemmStridedBatched",
                          "GemmStridedBatchedEx"], p=[0.15, 0.15, 0.35, 0.1, 0.1, 0.15]))
    if entry.startswith("S"):
        ab, ct = "f32", "f32"
    elif entry.startswith("H"):
        ab, ct = "f16", "f16"
    else:
        ab, ct = EX[r.integers(len(EX))]
    cls = str(r.choice(["decode", "tiles", "large", "longk"], p=[0.3, 0.4, 0.1, 0.2]))
    if cls == "decode":   # hipBLAS n = tokens (the engine's rows)
        m, n, k = int(r.integers(1, 3000)), int(r.integers(1, 65)), int(r.integers(1, 6000))
    elif cls == "tiles":
        m, n, k = int(r.integers(65, 1100)), int(r.integers(65, 1100)), int(r.integers(1, 2500))
    elif cls == "large":
        m, n, k = int(r.integers(2000, 4400)), int(r.integers(2000, 4400)), int(r.integers(64, 1100))
    else:
        m, n, k = int(r.integers(1, 300)), int(r.integers(1, 300)), int(r.integers(2048, 20000))
    aligned = r.random() < 0.65
    if aligned:
        m = -(-m // 8) * 8
        n = n if n <= 64 else -(-n // 8) * 8
        k = -(-k // 128) * 128 if r.random() < 0.7 else -(-k // 8) * 8

    def pad():
        if aligned:
            return 0 if r.random() < 0.7 else 8 * int(r.integers(1, 5))
        return 0 if r.random() < 0.5 else int(r.integers(1, 18))
    ops = ["N", "T", "C"]
    return dict(i=i, entry=entry, ab=ab, ct=ct, cls=cls, m=m, n=n, k=k, ta=ops[r.integers(3)], tb=ops[r.integers(3)],
                pa=pad(), pb=pad(), pc=pad(), batch=int(r.integers(2, 4)) if "Strided" in entry else 1,
                alpha=float(np.round(r.uniform(-2, 2), 3)),
                beta=0.0 if r.random() < 0.5 else float(np.round(r.uniform(-1.5, 1.5), 3)),
                device_scalars=bool(r.random() < 0.25))


CASES = [_draw(i) for i in range(NCASES)]


def _id(c):
    return f"{c['i']}_{c['entry']}_{c['ab']}-{c['ct']}_{c['ta']}{c['tb']}_m{c['m']}n{c['n']}k{c['k']}b{c['batch']}"


def _mats(r, nb, stride, rows, cols, ld, t, scale):
    """nb row-major rows x cols matrices (pitch ld, `stride` apart), NaN in
    every gap and padding."""
    buf = np.full(nb * stride, NAN[t], np.float32 if t == "f32" else np.uint16)
    for b in range(nb):
        vals = CONV[t]((r.standard_normal(rows * cols) * scale).astype(np.float32)).reshape(rows, cols)
        buf[b * stride: b * stride + rows * ld].reshape(rows, ld)[:, :cols] = vals
    return buf


@pytest.fixture(scope="module")
def handle():
    from gpu_helpers import Handle
    h = Handle()
    yield h
    h.close()


@pytest.mark.parametrize("c", CASES, ids=_id)
def test_random_hipblas(handle, c):
    import torch
    import vkblas_amd as vk
    from vkblas_amd import hipblas_abi as hb
    from gpu_helpers import normwise, f32_bound, F16_BOUND, BF16_BOUND
    print(f"[case] hipblas random {_id(c)} {c}", flush=True)
    TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
    HT = {"f32": hb.HIP_R_32F, "f16": hb.HIP_R_16F, "bf16": hb.HIP_R_16BF}
    DT = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    OP = {"N": hb.HIPBLAS_OP_N, "T": hb.HIPBLAS_OP_T, "C": hb.HIPBLAS_OP_C}
    ab, ct, m, n, k, nb = c["ab"], c["ct"], c["m"], c["n"], c["k"], c["batch"]
    ta, tb = int(c["ta"] != "N"), int(c["tb"] != "N")
    r = np.random.default_rng(9000 + c["i"])
    # column-major A: m x k (lda >= m), or k x m under T / C: in row-major
    # terms k rows of m (or m rows of k), pitch lda; likewise B and C
    a_rows, a_cols = (m, k) if ta else (k, m)
    b_rows, b_cols = (k, n) if tb else (n, k)
    lda, ldb, ldc = a_cols + c["pa"], b_cols + c["pb"], m + c["pc"]
    gap = 8 if nb > 1 else 0
    sa, sb, sc = a_rows * lda + gap, b_rows * ldb + gap, n * ldc + gap
    A = _mats(r, nb, sa, a_rows, a_cols, lda, ab, 1.0)
    B = _mats(r, nb, sb, b_rows, b_cols, ldb, ab, 0.05)
    C0 = _mats(r, nb, sc, n, m, ldc, ct, 1.0)
    gpu_c = C0.copy()
    if c["beta"] == 0.0:
        gpu_c[:] = NAN[ct]

    def dev(x, t):
        x = np.ascontiguousarray(x)
        return torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x).view(TD[t]).to("cuda:0")
    dA, dB, dC = dev(A, ab), dev(B, ab), dev(gpu_c, ct)
    half_scalars = c["entry"].startswith("H")
    if c["device_scalars"]:
        sdt = torch.float16 if half_scalars else torch.float32
        dsc = torch.tensor([c["alpha"], c["beta"]], dtype=sdt, device="cuda:0")
        es = 2 if half_scalars else 4
        pal, pbe = ctypes.c_void_p(dsc.data_ptr()), ctypes.c_void_p(dsc.data_ptr() + es)
        handle.set_pointer_mode(hb.HIPBLAS_POINTER_MODE_DEVICE)
    elif half_scalars:
        ha, hbt = [ctypes.c_uint16(int(np.array([v], np.float16).view(np.uint16)[0])) for v in (c["alpha"], c["beta"])]
        pal, pbe = ctypes.byref(ha), ctypes.byref(hbt)
    else:
        ha, hbt = ctypes.c_float(c["alpha"]), ctypes.c_float(c["beta"])
        pal, pbe = ctypes.byref(ha), ctypes.byref(hbt)
    handle.set_stream(torch.cuda.current_stream().cuda_stream)
    # a marker call whose path differs from this call's: if the hipBLAS call
    # were forwarded, the last path would stay the marker's
    pl = vk.plan(DT[ab], DT[ct], tb, ta, n, m, k, ldb, lda, ldc, nb)
    mk = torch.zeros(64 * 64, dtype=torch.float32, device="cuda:0")
    if pl.path == vk.PATH_TILE64:
        x = torch.zeros(8192, dtype=torch.float16, device="cuda:0")
        vk.gemm_async(vk.DT_F16, vk.DT_F16, vk.OP_N, vk.OP_T, 1, 8, 1024, 1.0, x.data_ptr(), 1024, x.data_ptr(), 1024,
                      0.0, mk.data_ptr(), 8)
        marker = vk.PATH_SKINNY
    else:
        x = torch.zeros(2 * 96 * 8, dtype=torch.float32, device="cuda:0")
        mk = torch.zeros(96 * 96, dtype=torch.float32, device="cuda:0")
        vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, vk.OP_N, 96, 96, 8, 1.0, x.data_ptr(), 8,
                      x.data_ptr() + 4 * 96 * 8, 96, 0.0, mk.data_ptr(), 96)
        marker = vk.PATH_TILE64
    assert vk.last_path() == marker
    try:
        a = handle.abi
        e = c["entry"]
        if e == "Sgemm" or e == "Hgemm":
            st = getattr(a, "hipblas" + e)(handle.h, OP[c["ta"]], OP[c["tb"]], m, n, k, pal, dA.data_ptr(), lda,
                                            dB.data_ptr(), ldb, pbe, dC.data_ptr(), ldc)
        elif e in ("SgemmStridedBatched", "HgemmStridedBatched"):
            st = getattr(a, "hipblas" + e)(handle.h, OP[c["ta"]], OP[c["tb"]], m, n, k, pal, dA.data_ptr(), lda, sa,
                                            dB.data_ptr(), ldb, sb, pbe, dC.data_ptr(), ldc, sc, nb)
        elif e == "GemmEx":
            st = a.hipblasGemmEx(handle.h, OP[c["ta"]], OP[c["tb"]], m, n, k, pal, dA.data_ptr(), HT[ab], lda,
                                 dB.data_ptr(), HT[ab], ldb, pbe, dC.data_ptr(), HT[ct], ldc, hb.HIPBLAS_COMPUTE_32F,
                                 hb.HIPBLAS_GEMM_DEFAULT)
        else:
            st = a.hipblasGemmStridedBatchedEx(handle.h, OP[c["ta"]], OP[c["tb"]], m, n, k, pal, dA.data_ptr(), HT[ab],
                                               lda, sa, dB.data_ptr(), HT[ab], ldb, sb, pbe, dC.data_ptr(), HT[ct],
                                               ldc, sc, nb, hb.HIPBLAS_COMPUTE_32F, hb.HIPBLAS_GEMM_DEFAULT)
        torch.cuda.synchronize()
    finally:
        if c["device_scalars"]:
            handle.set_pointer_mode(hb.HIPBLAS_POINTER_MODE_HOST)
    assert st == hb.HIPBLAS_STATUS_SUCCESS
    assert vk.last_path() == pl.path, "the call was forwarded"
    got_all = dC.cpu()
    got_all = got_all.view(torch.int16).numpy().view(np.uint16) if ct != "f32" else got_all.numpy()
    rows = oracle.sample_rows(n, 16) if m * n * k > 64 * 1024 * 1024 else None
    sel = np.arange(n) if rows is None else rows
    bound = f32_bound(k) if (ab, ct) == ("f32", "f32") else (BF16_BOUND if ct == "bf16" else F16_BOUND)
    for b in range(nb):
        want = C0[b * sc: b * sc + n * ldc].copy()
        oracle.ref_gemm_epi_rm(ab, ct, tb, ta, n, m, k, np.ascontiguousarray(B[b * sb:(b + 1) * sb]), ldb,
                               np.ascontiguousarray(A[b * sa:(b + 1) * sa]), lda, c["alpha"], c["beta"],
                               want.copy(), ldc, want, ldc, None, rows=rows)
        got = got_all[b * sc: b * sc + n * ldc]
        g = BACK[ct](np.stack([got[j * ldc: j * ldc + m] for j in sel]))
        w = BACK[ct](np.stack([want[j * ldc: j * ldc + m] for j in sel]))
        assert np.all(np.isfinite(g)), f"batch {b}: non-finite output"
        err = normwise(g, w)
        assert err <= bound, f"batch {b}: normwise {err:.3g} > {bound:.3g}"


# hipblasGemmEx type and compute codes: every fp32-compute code (32F, its
# PEDANTIC and FAST_16F / FAST_16BF / FAST_TF32 forms: full fp32 arithmetic is
# an allowed implementation of each), COMPUTE_16F with half scalars for
# fp16 -> fp16, and the pre-3.0 hipblasDatatype_t values (150 = R_16F,
# 151 = R_32F, 168 = R_16B, also as compute types) that the reference
# accepted (src/vkblas_hipblas.c:280-284).  Each call computed here (the
# marker call's path replaced) and checked against the oracle.
COMPUTE = {"16F": 0, "32F": 2, "32F_PEDANTIC": 3, "32F_FAST_16F": 4, "32F_FAST_16BF": 5, "32F_FAST_TF32": 6,
           "legacy_16F": 150, "legacy_32F": 151}
MODERN = {"f32": 0, "f16": 2, "bf16": 14}
LEGACY = {"f32": 151, "f16": 150, "bf16": 168}
CT_CASES = []
for comp in ("32F", "32F_PEDANTIC", "32F_FAST_16F", "32F_FAST_16BF", "32F_FAST_TF32", "legacy_32F"):
    for ab, ct in (("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32"), ("f32", "f32"),
                   ("f32", "f16"), ("f32", "bf16")):
        CT_CASES.append((ab, ct, comp, "modern"))
    CT_CASES.append(("f16", "f16", comp, "legacy"))
CT_CASES += [("f16", "f16", "16F", "modern"), ("f16", "f16", "16F", "legacy"), ("f16", "f16", "legacy_16F", "legacy"),
             ("bf16", "bf16", "32F", "legacy"), ("bf16", "f32", "legacy_32F", "legacy"), ("f32", "f32", "32F", "legacy")]


@pytest.mark.parametrize("case", CT_CASES, ids=lambda c: f"{c[0]}-{c[1]}_{c[2]}_{c[3]}")
def test_gemmex_compute_and_type_codes(handle, case):
    import torch
    import vkblas_amd as vk
    from vkblas_amd import hipblas_abi as hb
    from gpu_helpers import normwise, f32_bound, F16_BOUND, BF16_BOUND
    ab, ct, comp, enums = case
    print(f"[case] gemmex codes {case}", flush=True)
    codes = LEGACY if enums == "legacy" else MODERN
    m, n, k, ta, tb = 296, 200, 264, 1, 0
    r = np.random.default_rng(4242)
    lda, ldb, ldc = k, k, m
    A = _mats(r, 1, m * lda, m, k, lda, ab, 1.0)       # A stored k x m column-major (T): m rows of k
    B = _mats(r, 1, n * ldb, n, k, ldb, ab, 0.05)      # B stored k x n column-major (N): n rows of k
    C = _mats(r, 1, n * ldc, n, m, ldc, ct, 1.0)
    TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}

    def dev(x, t):
        return torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x).view(TD[t]).to("cuda:0")
    dA, dB, dC = dev(A, ab), dev(B, ab), dev(C, ct)
    alpha, beta = 0.75, -0.5
    if COMPUTE[comp] in (0, 150):   # half scalars
        sa, sb = [ctypes.c_uint16(int(np.array([v], np.float16).view(np.uint16)[0])) for v in (alpha, beta)]
    else:
        sa, sb = ctypes.c_float(alpha), ctypes.c_float(beta)
    dt = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    pl = vk.plan(dt[ab], dt[ct], tb, ta, n, m, k, ldb, lda, ldc)
    x = torch.zeros(65 * 64, dtype=torch.float16, device="cuda:0")
    w = torch.zeros(64 * 64, dtype=torch.float16, device="cuda:0")
    y = torch.zeros(65 * 64, dtype=torch.float16, device="cuda:0")
    rows_mk = 2 if pl.path != vk.PATH_SKINNY else 65
    vk.gemm_async(vk.DT_F16, vk.DT_F16, 0, 1 if rows_mk == 2 else 0, rows_mk, 64, 64, 1.0, x.data_ptr(), 64,
                  w.data_ptr(), 64, 0.0, y.data_ptr(), 64)
    torch.cuda.synchronize()
    marker = vk.last_path()
    handle.set_stream(torch.cuda.current_stream().cuda_stream)
    st = handle.abi.hipblasGemmEx(handle.h, hb.HIPBLAS_OP_T, hb.HIPBLAS_OP_N, m, n, k, ctypes.byref(sa), dA.data_ptr(),
                                  codes[ab], lda, dB.data_ptr(), codes[ab], ldb, ctypes.byref(sb), dC.data_ptr(),
                                  codes[ct], ldc, COMPUTE[comp], hb.HIPBLAS_GEMM_DEFAULT)
    torch.cuda.synchronize()
    assert st == hb.HIPBLAS_STATUS_SUCCESS
    assert vk.last_path() == pl.path != marker, "the call was forwarded"
    got = dC.cpu()
    got = got.view(torch.int16).numpy().view(np.uint16) if ct != "f32" else got.numpy()
    want = C.copy()
    oracle.ref_gemm_epi_rm(ab, ct, tb, ta, n, m, k, B, ldb, A, lda, alpha, beta, C.copy(), ldc, want, ldc, None)
    bound = f32_bound(k) if (ab, ct) == ("f32", "f32") else (BF16_BOUND if ct == "bf16" else F16_BOUND)
    g = BACK[ct](got.reshape(n, ldc)[:, :m])
    wv = BACK[ct](want.reshape(n, ldc)[:, :m])
    assert normwise(g, wv) <= bound
