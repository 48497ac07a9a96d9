"""The rocBLAS layer of libvkblas_hipblas.so: rocblas_gemm_ex and
rocblas_gemm_strided_batched_ex (reference src/vkblas_hipblas.c:802-955), the
calls PyTorch's hipBLAS backend makes for fp16 GEMMs.

A rocBLAS handle from the real librocblas (the one the process already loaded
with torch) drives this library's entry points through ctypes.  The oracle is
the fp16 / fp32 CPU restatement: a column-major rocBLAS call D = alpha op(A)
op(B) + beta C is the row-major engine call (op_a = transB, op_b = transA,
M = n, N = m, A = b, B = a), the mapping of src/vkblas_hipblas.c:187-189.
Bars: fp32 normwise <= 1e-5 sqrt(K), fp16 normwise <= 2e-3, bf16 results
<= 8e-3 (one bf16 ulp), fp32 results of bf16 inputs <= 2e-3.
"""
import ctypes

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

OP = {0: 111, 1: 112}            # rocblas_operation none / transpose
F16, F32, F64, BF16 = 150, 151, 152, 168   # rocblas_datatype
HOST, DEVICE = 0, 1              # rocblas_pointer_mode

_vp, _i, _i64, _u32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint32


class RocblasHandle:
    def __init__(self):
        import torch  # noqa: F401  (loads the process's librocblas)
        import vkblas_amd as vk
        self.lib = vk.load()
        self.real = ctypes.CDLL("librocblas.so.5")
        self.h = _vp()
        assert self.real.rocblas_create_handle(ctypes.byref(self.h)) == 0
        L = self.lib
        L.rocblas_gemm_ex.restype = _i
        L.rocblas_gemm_ex.argtypes = [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp, _i, _i, _vp, _vp, _i, _i,
                                      _vp, _i, _i, _i, _i, ctypes.c_int32, _u32]
        L.rocblas_gemm_strided_batched_ex.restype = _i
        L.rocblas_gemm_strided_batched_ex.argtypes = [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _i64, _vp, _i, _i,
                                                      _i64, _vp, _vp, _i, _i, _i64, _vp, _i, _i, _i64, _i, _i, _i,
                                                      ctypes.c_int32, _u32]
        L.rocblas_gemm_batched_ex.restype = _i
        L.rocblas_gemm_batched_ex.argtypes = [_vp, _i, _i, _i, _i, _i, _vp, _vp, _i, _i, _vp, _i, _i, _vp, _vp, _i,
                                              _i, _vp, _i, _i, _i, _i, _i, ctypes.c_int32, _u32]

    def set_stream(self, s):
        assert self.real.rocblas_set_stream(self.h, _vp(s)) == 0

    def set_pointer_mode(self, mode):
        assert self.real.rocblas_set_pointer_mode(self.h, mode) == 0

    def close(self):
        self.real.rocblas_destroy_handle(self.h)


@pytest.fixture(scope="module")
def rh():
    import torch
    h = RocblasHandle()
    h.set_stream(torch.cuda.current_stream().cuda_stream)
    yield h
    h.close()


def _rng_f16(seed, n, scale=1.0):
    r = np.random.default_rng(seed)
    return (r.standard_normal(n) * scale).astype(np.float16).view(np.uint16)


def _expected(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, ctype):
    """column-major rocBLAS semantics via the row-major engine oracle"""
    out = C.copy()
    if ctype == F16:
        oracle.ref_gemm_f16_rm(tb, ta, n, m, k, B, ldb, A, lda, alpha, beta, out, ldc)
    else:
        oracle.ref_gemm_f16f32_rm(tb, ta, n, m, k, B, ldb, A, lda, alpha, beta, out, ldc)
    return out


def _cols(buf, m, n, ld):
    return np.concatenate([buf[j * ld: j * ld + m] for j in range(n)])


CASES = [(ta, tb, m, n, k, alpha, beta, ct)
         for (m, n, k) in ((64, 48, 40), (257, 129, 65), (256, 256, 256), (8, 4096, 512))
         for ta in (0, 1) for tb in (0, 1)
         for (alpha, beta) in ((1.0, 0.0), (0.5, -0.25))
         for ct in (F16, F32)]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{'NT'[c[0]]}{'NT'[c[1]]}_{c[2]}x{c[3]}x{c[4]}_a{c[5]}_b{c[6]}_"
                                                     f"{'f16' if c[7] == F16 else 'f32'}")
def test_gemm_ex_f16(rh, case):
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND, fbox
    ta, tb, m, n, k, alpha, beta, ct = case
    print(f"[case] rocblas_gemm_ex f16 {case}", flush=True)
    lda = (k if ta else m) + 1
    ldb = (n if tb else k) + 2
    ldc = m + 3
    A = _rng_f16(1, lda * (m if ta else k), 1 / np.sqrt(k))
    B = _rng_f16(2, ldb * (k if tb else n))
    C = _rng_f16(3, ldc * n) if ct == F16 else np.random.default_rng(3).standard_normal(ldc * n).astype(np.float32)
    want = _expected(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc, ct)
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    st = rh.lib.rocblas_gemm_ex(rh.h, OP[ta], OP[tb], m, n, k, fbox(alpha), dA.data_ptr(), F16, lda, dB.data_ptr(),
                                F16, ldb, fbox(beta), dC.data_ptr(), ct, ldc, dC.data_ptr(), ct, ldc, F32, 0, 0, 0)
    assert st == 0
    got = to_host(dC)
    if ct == F16:
        assert normwise(oracle.h2f(_cols(got, m, n, ldc)), oracle.h2f(_cols(want, m, n, ldc))) <= F16_BOUND
    else:
        assert normwise(_cols(got, m, n, ldc), _cols(want, m, n, ldc)) <= F16_BOUND
    pad = np.ones(got.size, bool)
    for j in range(n):
        pad[j * ldc: j * ldc + m] = False
    assert np.array_equal(got[pad], C[pad])   # rows m..ldc-1 of each column untouched


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 1), (0, 1), (1, 0)])
def test_gemm_ex_f32(rh, ta, tb):
    from gpu_helpers import to_dev, to_host, normwise, f32_bound, fbox
    m, n, k = 300, 200, 150
    print(f"[case] rocblas_gemm_ex f32 {ta}{tb}", flush=True)
    lda, ldb, ldc = (k if ta else m), (n if tb else k), m
    A, B, C = oracle.fill_test_gemm(5 + 2 * ta + tb, lda * (m if ta else k), ldb * (k if tb else n), ldc * n)
    want = C.copy()
    oracle.ref_gemm_cm(ta, tb, m, n, k, 0.5, A, lda, B, ldb, 0.7, want, ldc)
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    st = rh.lib.rocblas_gemm_ex(rh.h, OP[ta], OP[tb], m, n, k, fbox(0.5), dA.data_ptr(), F32, lda, dB.data_ptr(),
                                F32, ldb, fbox(0.7), dC.data_ptr(), F32, ldc, dC.data_ptr(), F32, ldc, F32, 0, 0, 0)
    assert st == 0
    assert normwise(to_host(dC), want) <= f32_bound(k)


def test_separate_d_and_device_scalars(rh):
    """D != C (C copied into D first), scalars in device memory."""
    import torch
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND
    m, n, k = 130, 70, 96
    print("[case] rocblas_gemm_ex separate D, device pointer mode", flush=True)
    A = _rng_f16(11, m * k, 1 / np.sqrt(k))
    B = _rng_f16(12, k * n)
    C = _rng_f16(13, m * n)
    want = _expected(0, 0, m, n, k, 2.0, A, m, B, k, 0.5, C, m, F16)
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    dD = torch.full((m * n,), float("nan"), dtype=torch.float16, device="cuda:0")
    scal = torch.tensor([2.0, 0.5], dtype=torch.float32, device="cuda:0")
    # a decode call first: a call the engine computes replaces its path as
    # vkblas_last_path, a forwarded one leaves it
    import vkblas_amd as vk
    x = torch.zeros(2 * 64, dtype=torch.float16, device="cuda:0")
    w = torch.zeros(64 * 64, dtype=torch.float16, device="cuda:0")
    vk.gemm_async(vk.DT_F16, vk.DT_F16, 0, 1, 2, 64, 64, 1.0, x.data_ptr(), 64, w.data_ptr(), 64, 0.0,
                  x.data_ptr(), 64)
    torch.cuda.synchronize()
    assert vk.last_path() == vk.PATH_SKINNY
    rh.set_pointer_mode(DEVICE)
    try:
        st = rh.lib.rocblas_gemm_ex(rh.h, OP[0], OP[0], m, n, k, scal.data_ptr(), dA.data_ptr(), F16, m,
                                    dB.data_ptr(), F16, k, scal.data_ptr() + 4, dC.data_ptr(), F16, m, dD.data_ptr(),
                                    F16, m, F32, 0, 0, 0)
    finally:
        rh.set_pointer_mode(HOST)
    assert st == 0
    assert vk.last_path() != vk.PATH_SKINNY, "the call was forwarded"
    assert normwise(oracle.h2f(to_host(dD)), oracle.h2f(want)) <= F16_BOUND
    assert np.array_equal(to_host(dC), C)   # C is read-only


def test_strided_batched_f16(rh):
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND, fbox
    m, n, k, nb = 96, 80, 64, 3
    print("[case] rocblas_gemm_strided_batched_ex f16", flush=True)
    sa, sb, sc = m * k + 7, k * n + 5, m * n + 3
    A = _rng_f16(21, sa * nb, 1 / np.sqrt(k))
    B = _rng_f16(22, sb * nb)
    C = _rng_f16(23, sc * nb)
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    st = rh.lib.rocblas_gemm_strided_batched_ex(rh.h, OP[1], OP[0], m, n, k, fbox(1.0), dA.data_ptr(), F16, k, sa,
                                                dB.data_ptr(), F16, k, sb, fbox(1.0), dC.data_ptr(), F16, m, sc,
                                                dC.data_ptr(), F16, m, sc, nb, F32, 0, 0, 0)
    assert st == 0
    got = to_host(dC)
    for i in range(nb):
        want = _expected(1, 0, m, n, k, 1.0, A[i * sa:], k, B[i * sb:], k, 1.0, C[i * sc: i * sc + m * n].copy(), m,
                         F16)
        assert normwise(oracle.h2f(got[i * sc: i * sc + m * n]), oracle.h2f(want)) <= F16_BOUND


BF_CASES = [(ta, tb, m, n, k, ct) for (m, n, k) in ((64, 48, 40), (257, 129, 65), (512, 256, 256), (8, 1024, 512))
            for ta in (0, 1) for tb in (0, 1) for ct in (BF16, F32)]


@pytest.mark.parametrize("case", BF_CASES, ids=lambda c: f"{'NT'[c[0]]}{'NT'[c[1]]}_{c[2]}x{c[3]}x{c[4]}_"
                                                          f"{'bf16' if c[5] == BF16 else 'f32'}")
def test_gemm_ex_bf16(rh, case):
    """bf16 data (PyTorch's bf16 matmul path): computed by this library, not forwarded."""
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND, BF16_BOUND, fbox
    ta, tb, m, n, k, ct = case
    print(f"[case] rocblas_gemm_ex bf16 {case}", flush=True)
    lda = (k if ta else m) + 2
    ldb = (n if tb else k) + 1
    ldc = m + 1
    r = np.random.default_rng(7 + m + k)
    A = oracle.f2bf_rne((r.standard_normal(lda * (m if ta else k)) / np.sqrt(k)).astype(np.float32))
    B = oracle.f2bf_rne(r.standard_normal(ldb * (k if tb else n)).astype(np.float32))
    C32 = r.standard_normal(ldc * n).astype(np.float32)
    C = oracle.f2bf_rne(C32) if ct == BF16 else C32
    want = C.copy()
    fn = oracle.ref_gemm_bf16_rm if ct == BF16 else oracle.ref_gemm_bf16f32_rm
    fn(tb, ta, n, m, k, B, ldb, A, lda, 1.5, -0.5, want, ldc)
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    st = rh.lib.rocblas_gemm_ex(rh.h, OP[ta], OP[tb], m, n, k, fbox(1.5), dA.data_ptr(), BF16, lda, dB.data_ptr(),
                                BF16, ldb, fbox(-0.5), dC.data_ptr(), ct, ldc, dC.data_ptr(), ct, ldc, F32, 0, 0, 0)
    assert st == 0
    got = to_host(dC)
    g, w = _cols(got, m, n, ldc), _cols(want, m, n, ldc)
    if ct == BF16:
        assert normwise(oracle.bf2f(g), oracle.bf2f(w)) <= BF16_BOUND
    else:
        assert normwise(g, w) <= F16_BOUND
    pad = np.ones(got.size, bool)
    for j in range(n):
        pad[j * ldc: j * ldc + m] = False
    assert np.array_equal(got[pad], C[pad])


def test_strided_batched_bf16(rh):
    from gpu_helpers import to_dev, to_host, normwise, BF16_BOUND, fbox
    m, n, k, nb = 96, 80, 64, 3
    print("[case] rocblas_gemm_strided_batched_ex bf16", flush=True)
    sa, sb, sc = m * k + 7, k * n + 5, m * n + 3
    r = np.random.default_rng(24)
    A = oracle.f2bf_rne((r.standard_normal(sa * nb) / 8).astype(np.float32))
    B = oracle.f2bf_rne(r.standard_normal(sb * nb).astype(np.float32))
    C = oracle.f2bf_rne(r.standard_normal(sc * nb).astype(np.float32))
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    st = rh.lib.rocblas_gemm_strided_batched_ex(rh.h, OP[1], OP[0], m, n, k, fbox(1.0), dA.data_ptr(), BF16, k, sa,
                                                dB.data_ptr(), BF16, k, sb, fbox(1.0), dC.data_ptr(), BF16, m, sc,
                                                dC.data_ptr(), BF16, m, sc, nb, F32, 0, 0, 0)
    assert st == 0
    got = to_host(dC)
    for i in range(nb):
        want = C[i * sc: i * sc + m * n].copy()
        oracle.ref_gemm_bf16_rm(0, 1, n, m, k, B[i * sb:], k, A[i * sa:], k, 1.0, 1.0, want, m)
        assert normwise(oracle.bf2f(got[i * sc: i * sc + m * n]), oracle.bf2f(want)) <= BF16_BOUND


def test_forwarded_calls_still_work(rh):
    """fp64 (no kernels here) and m == 0 (quick return) reach the real rocBLAS."""
    import torch
    from gpu_helpers import fbox
    print("[case] rocblas_gemm_ex forwarded f64 / m=0", flush=True)
    m = n = k = 64
    a = torch.randn(m, k, device="cuda:0", dtype=torch.float64)
    b = torch.randn(k, n, device="cuda:0", dtype=torch.float64)
    c = torch.zeros(n, m, device="cuda:0", dtype=torch.float64)
    one, zero = ctypes.byref(ctypes.c_double(1.0)), ctypes.byref(ctypes.c_double(0.0))
    # column-major: A^T as stored (k x m col-major = a row-major), C = a @ b in row-major = (b^T a^T)^T
    st = rh.lib.rocblas_gemm_ex(rh.h, OP[0], OP[0], n, m, k, one, b.data_ptr(), F64, n, a.data_ptr(), F64,
                                k, zero, c.data_ptr(), F64, n, c.data_ptr(), F64, n, F64, 0, 0, 0)
    assert st == 0
    torch.cuda.synchronize()
    ref = a.cpu() @ b.cpu()
    got = c.cpu().reshape(m, n)
    assert float((got - ref).abs().max() / ref.abs().max()) < 1e-12
    st = rh.lib.rocblas_gemm_ex(rh.h, OP[0], OP[0], 0, n, k, fbox(1.0), b.data_ptr(), F16, n, a.data_ptr(), F16,
                                k, fbox(0.0), c.data_ptr(), F16, n, c.data_ptr(), F16, n, F32, 0, 0, 0)
    assert st == 0


@pytest.mark.parametrize("dt", [F16, BF16])
def test_gemm_batched_ex_ptr_array(rh, dt):
    """rocblas_gemm_batched_ex: device arrays of matrix pointers (D == C computed here)."""
    import torch
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND, BF16_BOUND, fbox
    m, n, k, nb = 120, 72, 88, 3
    print(f"[case] rocblas_gemm_batched_ex {dt}", flush=True)
    conv = oracle.f2bf_rne if dt == BF16 else oracle.f2h_rne
    dec = oracle.bf2f if dt == BF16 else oracle.h2f
    ref = oracle.ref_gemm_bf16_rm if dt == BF16 else oracle.ref_gemm_f16_rm
    r = np.random.default_rng(31)
    As = [conv((r.standard_normal(m * k) / 8).astype(np.float32)) for _ in range(nb)]
    Bs = [conv(r.standard_normal(k * n).astype(np.float32)) for _ in range(nb)]
    Cs = [conv(r.standard_normal(m * n).astype(np.float32)) for _ in range(nb)]
    dA = [to_dev(a) for a in As]
    dB = [to_dev(b) for b in Bs]
    dC = [to_dev(c) for c in Cs]
    pa = torch.tensor([t.data_ptr() for t in dA], dtype=torch.int64, device="cuda:0")
    pb = torch.tensor([t.data_ptr() for t in dB], dtype=torch.int64, device="cuda:0")
    pc = torch.tensor([t.data_ptr() for t in dC], dtype=torch.int64, device="cuda:0")
    st = rh.lib.rocblas_gemm_batched_ex(rh.h, OP[0], OP[1], m, n, k, fbox(1.0), pa.data_ptr(), dt, m, pb.data_ptr(),
                                        dt, n, fbox(0.5), pc.data_ptr(), dt, m, pc.data_ptr(), dt, m, nb, F32, 0, 0, 0)
    assert st == 0
    bound = BF16_BOUND if dt == BF16 else F16_BOUND
    for i in range(nb):
        want = Cs[i].copy()
        # column-major C = A op(B)^T with B (n x k) -> engine: op_a = transB = T, op_b = transA = N
        ref(1, 0, n, m, k, Bs[i], n, As[i], m, 1.0, 0.5, want, m)
        assert normwise(dec(to_host(dC[i])), dec(want)) <= bound


# Seeded random sweep: rocblas_gemm_ex / rocblas_gemm_strided_batched_ex with
# every type pair the layer computes, both transposes, decode-shaped and
# general shapes (aligned or ragged), padding, beta (0 over a NaN C), C == D
# or a separate D, host or device scalars, strided batches; each call
# asserted computed (a marker call on another path first) and checked
# against the oracle (oracle.ref_gemm_epi_rm on the row-major mapping).
RT = {"f16": F16, "f32": F32, "bf16": BF16}
SW_TYPES = [("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32"), ("f32", "f32")]
SW_NAN = {"f32": np.float32(np.nan), "f16": np.uint16(0x7E00), "bf16": np.uint16(0x7FC0)}
SW_CONV = {"f32": lambda x: x.astype(np.float32), "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}
SW_BACK = {"f32": lambda x: x.astype(np.float32), "f16": oracle.h2f, "bf16": oracle.bf2f}


def _sw_case(i):
    r = np.random.default_rng(60000 + i)
    ab, ct = SW_TYPES[r.integers(len(SW_TYPES))]
    if r.random() < 0.3:
        m, n, k = int(r.integers(8, 4097)), int(r.integers(1, 17)), int(r.integers(8, 2049))
    else:
        m, n, k = int(r.integers(1, 700)), int(r.integers(1, 700)), int(r.integers(1, 1600))
    if r.random() < 0.6:
        m, k = -(-m // 8) * 8, -(-k // 8) * 8
        pads = tuple(int(8 * r.integers(0, 3)) for _ in range(4))
    else:
        pads = tuple(int(r.integers(0, 9)) for _ in range(4))
    return dict(ab=ab, ct=ct, ta=int(r.integers(2)), tb=int(r.integers(2)), m=m, n=n, k=k, pads=pads,
                alpha=float(np.round(r.uniform(-2, 2), 3)),
                beta=0.0 if r.random() < 0.5 else float(np.round(r.uniform(-1.5, 1.5), 3)),
                sep_d=bool(r.random() < 0.3), device=bool(r.random() < 0.25),
                batch=int(r.integers(2, 4)) if r.random() < 0.2 else 1)


SW_CASES = [_sw_case(i) for i in range(150)]


def _sw_mats(r, nb, stride, rows, cols, ld, t, scale):
    buf = np.full(nb * stride, SW_NAN[t], np.float32 if t == "f32" else np.uint16)
    for b in range(nb):
        vals = SW_CONV[t]((r.standard_normal(rows * cols) * scale).astype(np.float32)).reshape(rows, cols)
        buf[b * stride: b * stride + rows * ld].reshape(rows, ld)[:, :cols] = vals
    return buf


@pytest.mark.parametrize("c", SW_CASES, ids=[f"{i}" for i in range(len(SW_CASES))])
def test_gemm_ex_random_sweep(rh, c):
    import torch
    import vkblas_amd as vk
    from gpu_helpers import normwise, f32_bound, F16_BOUND, BF16_BOUND
    print(f"[case] rocblas sweep {c}", flush=True)
    ab, ct, m, n, k, ta, tb, nb = c["ab"], c["ct"], c["m"], c["n"], c["k"], c["ta"], c["tb"], c["batch"]
    r = np.random.default_rng(80000 + m + n + k)
    # column-major A: m x k (k x m under T): k rows of m in row-major terms
    a_rows, a_cols = (m, k) if ta else (k, m)
    b_rows, b_cols = (k, n) if tb else (n, k)
    lda, ldb, ldc, ldd = a_cols + c["pads"][0], b_cols + c["pads"][1], m + c["pads"][2], m + c["pads"][3]
    gap = 8 if nb > 1 else 0
    sa, sb, sc, sd = a_rows * lda + gap, b_rows * ldb + gap, n * ldc + gap, n * ldd + gap
    A = _sw_mats(r, nb, sa, a_rows, a_cols, lda, ab, 1.0)
    B = _sw_mats(r, nb, sb, b_rows, b_cols, ldb, ab, 0.05)
    C = _sw_mats(r, nb, sc, n, m, ldc, ct, 1.0)
    TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}

    def dev(x, t):
        return torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x).view(TD[t]).to("cuda:0")
    gpu_c = C.copy()
    if c["beta"] == 0.0 and not c["sep_d"]:
        gpu_c[:] = SW_NAN[ct]
    dA, dB, dC = dev(A, ab), dev(B, ab), dev(gpu_c, ct)
    D0 = np.full(nb * sd, SW_NAN[ct], np.float32 if ct == "f32" else np.uint16) if c["sep_d"] else None
    dD = dev(D0, ct) if c["sep_d"] else dC
    ldd_ = ldd if c["sep_d"] else ldc
    sd_ = sd if c["sep_d"] else sc
    pl = vk.plan({"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}[ab],
                 {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}[ct], tb, ta, n, m, k, ldb, lda, ldd_, nb)
    # the marker: 2 rows against W stored N x K (the decode kernels) or 65
    # against W stored K x N (a 64x64 tile), whichever this call does not take
    x = torch.zeros(65 * 64, dtype=torch.float16, device="cuda:0")
    w = torch.zeros(64 * 64, dtype=torch.float16, device="cuda:0")
    y = torch.zeros(65 * 64, dtype=torch.float16, device="cuda:0")
    rows_mk = 2 if pl.path != vk.PATH_SKINNY else 65
    vk.gemm_async(vk.DT_F16, vk.DT_F16, 0, 1 if rows_mk == 2 else 0, rows_mk, 64, 64, 1.0, x.data_ptr(), 64,
                  w.data_ptr(), 64, 0.0, y.data_ptr(), 64)
    torch.cuda.synchronize()
    marker = vk.last_path()
    assert marker == (vk.PATH_SKINNY if rows_mk == 2 else vk.PATH_TILE64)
    if c["device"]:
        sc_dev = torch.tensor([c["alpha"], c["beta"]], dtype=torch.float32, device="cuda:0")
        pa, pb = ctypes.c_void_p(sc_dev.data_ptr()), ctypes.c_void_p(sc_dev.data_ptr() + 4)
        rh.set_pointer_mode(DEVICE)
    else:
        ha, hb_ = ctypes.c_float(c["alpha"]), ctypes.c_float(c["beta"])
        pa, pb = ctypes.byref(ha), ctypes.byref(hb_)
    try:
        if nb == 1:
            st = rh.lib.rocblas_gemm_ex(rh.h, OP[ta], OP[tb], m, n, k, pa, dA.data_ptr(), RT[ab], lda, dB.data_ptr(),
                                        RT[ab], ldb, pb, dC.data_ptr(), RT[ct], ldc, dD.data_ptr(), RT[ct], ldd_, F32,
                                        0, 0, 0)
        else:
            st = rh.lib.rocblas_gemm_strided_batched_ex(rh.h, OP[ta], OP[tb], m, n, k, pa, dA.data_ptr(), RT[ab], lda,
                                                        sa, dB.data_ptr(), RT[ab], ldb, sb, pb, dC.data_ptr(), RT[ct],
                                                        ldc, sc, dD.data_ptr(), RT[ct], ldd_, sd_, nb, F32, 0, 0, 0)
        torch.cuda.synchronize()
    finally:
        if c["device"]:
            rh.set_pointer_mode(HOST)
    assert st == 0
    assert vk.last_path() == pl.path != marker, "the call was forwarded"
    got = dD.cpu()
    got = got.view(torch.int16).numpy().view(np.uint16) if ct != "f32" else got.numpy()
    rows = oracle.sample_rows(n, 16) if m * n * k > 64 * 1024 * 1024 else None
    sel = np.arange(n) if rows is None else rows
    bound = f32_bound(k) if (ab, ct) == ("f32", "f32") else (BF16_BOUND if ct == "bf16" else F16_BOUND)
    for b in range(nb):
        want = np.full(n * ldd_, SW_NAN[ct], got.dtype)
        oracle.ref_gemm_epi_rm(ab, ct, tb, ta, n, m, k, np.ascontiguousarray(B[b * sb:(b + 1) * sb]), ldb,
                               np.ascontiguousarray(A[b * sa:(b + 1) * sa]), lda, c["alpha"], c["beta"],
                               np.ascontiguousarray(C[b * sc: b * sc + n * ldc]), ldc, want, ldd_, None, rows=rows)
        gb = got[b * sd_: b * sd_ + n * ldd_]
        g = SW_BACK[ct](np.stack([gb[j * ldd_: j * ldd_ + m] for j in sel]))
        wv = SW_BACK[ct](np.stack([want[j * ldd_: j * ldd_ + m] for j in sel]))
        assert np.all(np.isfinite(g)), f"batch {b}"
        err = normwise(g, wv)
        assert err <= bound, f"batch {b}: {err:.3g}"
    if c["sep_d"]:
        assert np.array_equal(dC.cpu().view(torch.int16 if ct != "f32" else torch.int32).numpy().view(
            np.uint16 if ct != "f32" else np.uint32), gpu_c.view(np.uint16 if ct != "f32" else np.uint32)), \
            "C was written"
