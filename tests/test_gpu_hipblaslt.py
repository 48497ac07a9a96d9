"""hipblasLtMatmul through this library's entry point, with descriptors and
layouts made by the real hipBLASLt the process uses (PyTorch's copy).

hipBLASLt is column-major: D(m x n) = alpha op(A) op(B) + beta C (+ bias[row]
with HIPBLASLT_EPILOGUE_BIAS).  Cases: every type combination the library
computes, all four transposes, the bias epilogue (bias type unset = D's
type, and explicit fp32 for 16-bit D), C == D and a separate C with its own
leading dimension, strided batches, host and device alpha / beta.  The
results are checked against the oracle's epilogue restatement
(oracle.ref_gemm_epi_rm on the row-major mapping D' = op(B)' op(A)').  That
the library computed a call (rather than forwarding it) shows in
vkblas_last_path; calls it does not compute (activation epilogues, scale
pointers) must be forwarded and leave it unchanged.  No reference
counterpart: PyTorch on gfx950 reaches these entry points where the
reference's PyTorch reached its hipBLAS ones (reference src/vkblas_hipblas.c:
802-808, test/test_torch.py:65-73).
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

HIP_R_32F, HIP_R_16F, HIP_R_16BF = 0, 2, 14
HIPBLAS_OP_N, HIPBLAS_OP_T = 111, 112
HIPBLAS_COMPUTE_32F = 2
EPI_DEFAULT, EPI_RELU, EPI_BIAS, EPI_GELU_BIAS = 1, 2, 4, 36
A_TRANSA, A_TRANSB, A_EPILOGUE, A_BIAS_POINTER, A_BIAS_TYPE, A_A_SCALE, A_POINTER_MODE = 0, 1, 2, 3, 4, 5, 13
L_BATCH, L_STRIDE = 0, 1
TYPES = {"f32": (HIP_R_32F, torch.float32), "f16": (HIP_R_16F, torch.float16), "bf16": (HIP_R_16BF, torch.bfloat16)}
CONV = {"f32": lambda x: x.astype(np.float32), "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}
BACK = {"f32": lambda x: x.astype(np.float32), "f16": oracle.h2f, "bf16": oracle.bf2f}
_vp = ctypes.c_void_p


class Lt:
    """The real hipBLASLt (the instance PyTorch loaded: its handle) and this
    library's interposed entry points (everything a caller that has the
    library preloaded would reach by name)."""

    def __init__(self):
        import vkblas_amd as vk
        self.real = ctypes.CDLL("libhipblaslt.so.1")
        self.ours = vk.load()
        r, o = self.real, self.ours
        r.hipblasLtCreate.argtypes = [ctypes.POINTER(_vp)]
        r.hipblasLtDestroy.argtypes = [_vp]
        o.hipblasLtMatrixLayoutCreate.argtypes = [ctypes.POINTER(_vp), ctypes.c_int, ctypes.c_uint64,
                                                  ctypes.c_uint64, ctypes.c_int64]
        o.hipblasLtMatrixLayoutDestroy.argtypes = [_vp]
        o.hipblasLtMatrixLayoutSetAttribute.argtypes = [_vp, ctypes.c_int, _vp, ctypes.c_size_t]
        o.hipblasLtMatmulDescSetAttribute.argtypes = [_vp, ctypes.c_int, _vp, ctypes.c_size_t]
        o.hipblasLtMatmulDescCreate.argtypes = [ctypes.POINTER(_vp), ctypes.c_int, ctypes.c_int]
        o.hipblasLtMatmulDescDestroy.argtypes = [_vp]
        o.hipblasLtMatmul.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                      ctypes.c_size_t, _vp]
        for f in (r.hipblasLtCreate, r.hipblasLtDestroy, o.hipblasLtMatrixLayoutCreate,
                  o.hipblasLtMatrixLayoutDestroy, o.hipblasLtMatrixLayoutSetAttribute,
                  o.hipblasLtMatmulDescSetAttribute, o.hipblasLtMatmulDescCreate, o.hipblasLtMatmulDescDestroy,
                  o.hipblasLtMatmul):
            f.restype = ctypes.c_int
        self.h = _vp()
        assert r.hipblasLtCreate(ctypes.byref(self.h)) == 0

    def layout(self, t, rows, cols, ld, batch=1, stride=0):
        lay = _vp()
        assert self.ours.hipblasLtMatrixLayoutCreate(ctypes.byref(lay), TYPES[t][0], rows, cols, ld) == 0
        if batch > 1:
            b, s = ctypes.c_int32(batch), ctypes.c_int64(stride)
            assert self.ours.hipblasLtMatrixLayoutSetAttribute(lay, L_BATCH, ctypes.byref(b), 4) == 0
            assert self.ours.hipblasLtMatrixLayoutSetAttribute(lay, L_STRIDE, ctypes.byref(s), 8) == 0
        return lay

    def desc(self, ta, tb, epilogue=EPI_DEFAULT, bias=None, bias_type=None, pmode=0, scale_ptr=None):
        d = _vp()
        assert self.ours.hipblasLtMatmulDescCreate(ctypes.byref(d), HIPBLAS_COMPUTE_32F, HIP_R_32F) == 0

        def set_(attr, val):
            assert self.ours.hipblasLtMatmulDescSetAttribute(d, attr, ctypes.byref(val), ctypes.sizeof(val)) == 0
        set_(A_TRANSA, ctypes.c_int32(HIPBLAS_OP_T if ta else HIPBLAS_OP_N))
        set_(A_TRANSB, ctypes.c_int32(HIPBLAS_OP_T if tb else HIPBLAS_OP_N))
        set_(A_EPILOGUE, ctypes.c_uint32(epilogue))
        if bias is not None:
            set_(A_BIAS_POINTER, _vp(bias))
        if bias_type is not None:
            set_(A_BIAS_TYPE, ctypes.c_int32(TYPES[bias_type][0]))
        if pmode:
            set_(A_POINTER_MODE, ctypes.c_int32(pmode))
        if scale_ptr is not None:
            set_(A_A_SCALE, _vp(scale_ptr))
        return d


@pytest.fixture(scope="module")
def lt():
    return Lt()


def _u(seed, n, s=1.0):
    return (np.random.default_rng(seed).uniform(-1, 1, n) * s).astype(np.float32)


def _dev(x, t):
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16)).view(TYPES[t][1]).to("cuda:0")
    return torch.from_numpy(x).to("cuda:0")


def _host(t):
    torch.cuda.synchronize()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()


def _mark_skinny(vk, skinny=True):
    """an engine call whose path a case does not take (the decode kernels, or
    with skinny=False a 64x64 tile): a forwarded call leaves that path as
    vkblas_last_path"""
    # 2 rows against W stored N x K: the decode kernels; 65 rows against W
    # stored K x N (more than its decode kernel takes): a 64x64 tile
    rows = 2 if skinny else 65
    x = torch.zeros(rows * 64, dtype=torch.float16, device="cuda:0")
    w = torch.zeros(64 * 64, dtype=torch.float16, device="cuda:0")
    y = torch.zeros(rows * 64, dtype=torch.float16, device="cuda:0")
    vk.gemm_async(vk.DT_F16, vk.DT_F16, 0, 1 if skinny else 0, rows, 64, 64, 1.0, x.data_ptr(), 64, w.data_ptr(),
                  64, 0.0, y.data_ptr(), 64)
    torch.cuda.synchronize()
    assert vk.last_path() == (vk.PATH_SKINNY if skinny else vk.PATH_TILE64)
    return vk.last_path()


def run_lt(lt, ab, dt, ta, tb, m, n, k, alpha, beta, bias_mode, sep_c, batch=1, pmode=0, pads=(2, 3, 4),
           decode=False):
    import vkblas_amd as vk
    from gpu_helpers import normwise, f32_bound, F16_BOUND, BF16_BOUND
    print(f"[case] lt {ab}>{dt} t={ta}{tb} {m}x{n}x{k} a={alpha} b={beta} bias={bias_mode} sepC={sep_c} "
          f"batch={batch} pmode={pmode}", flush=True)
    lda = (k if ta else m) + pads[0]
    ldb = (n if tb else k) + pads[1]
    ldd = m + pads[2]
    ldc = m + 6 if sep_c else ldd
    sa, sb, sd, sc = lda * (m if ta else k), ldb * (k if tb else n), ldd * n, ldc * n
    A = CONV[ab](_u(1 + m, sa * batch))
    B = CONV[ab](_u(2 + n, sb * batch))
    C = CONV[dt](_u(3, sc * batch))
    D0 = CONV[dt](_u(4, sd * batch)) if sep_c else C.copy()
    bias_t = None if bias_mode is None else (dt if bias_mode == "d" else bias_mode)
    bias = None if bias_t is None else CONV[bias_t](_u(5, m))
    want = D0.copy()
    for bi in range(batch):
        # column-major D(m x n) = row-major D'(n x m) = op(B)' op(A)'
        cin = (C if sep_c else want)[bi * sc:(bi + 1) * sc].copy()
        d = want[bi * sd:(bi + 1) * sd].copy()
        oracle.ref_gemm_epi_rm(ab, dt, tb, ta, n, m, k, np.ascontiguousarray(B[bi * sb:(bi + 1) * sb]), ldb,
                               np.ascontiguousarray(A[bi * sa:(bi + 1) * sa]), lda, alpha, beta, cin, ldc, d, ldd,
                               None if bias is None else BACK[bias_t](bias))
        want[bi * sd:(bi + 1) * sd] = d
    dA, dB, dD = _dev(A, ab), _dev(B, ab), _dev(D0, dt)
    dC = _dev(C, dt) if sep_c else dD
    dBias = _dev(bias, bias_t) if bias is not None else None
    la = lt.layout(ab, k if ta else m, m if ta else k, lda, batch, sa)
    lb = lt.layout(ab, n if tb else k, k if tb else n, ldb, batch, sb)
    lc = lt.layout(dt, m, n, ldc, batch, sc)
    ld = lt.layout(dt, m, n, ldd, batch, sd)
    desc = lt.desc(ta, tb, EPI_BIAS if bias is not None else EPI_DEFAULT,
                   None if dBias is None else dBias.data_ptr(),
                   None if bias_mode in (None, "d") else bias_t, pmode)
    if pmode:
        sc_dev = torch.tensor([alpha, beta], dtype=torch.float32, device="cuda:0")
        pa, pb = sc_dev.data_ptr(), sc_dev.data_ptr() + 4
    else:
        ha, hb = ctypes.c_float(alpha), ctypes.c_float(beta)
        pa, pb = ctypes.addressof(ha), ctypes.addressof(hb)
    marker = _mark_skinny(vk, skinny=not decode)
    st = lt.ours.hipblasLtMatmul(lt.h, desc, pa, dA.data_ptr(), la, dB.data_ptr(), lb, pb, dC.data_ptr(), lc,
                                 dD.data_ptr(), ld, None, None, 0, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    got = _host(dD)
    assert vk.last_path() != marker, "the call was forwarded"
    for lay in (la, lb, lc, ld):
        lt.ours.hipblasLtMatrixLayoutDestroy(lay)
    lt.ours.hipblasLtMatmulDescDestroy(desc)
    if sep_c:
        assert np.array_equal(_host(dC).view(np.uint8), C.view(np.uint8)), "C was written"
    bound = BF16_BOUND if dt == "bf16" else (f32_bound(k) if (ab, dt) == ("f32", "f32") else F16_BOUND)
    for bi in range(batch):
        g = BACK[dt](got[bi * sd:(bi + 1) * sd]).reshape(n, ldd)
        w = BACK[dt](want[bi * sd:(bi + 1) * sd]).reshape(n, ldd)
        assert np.array_equal(g[:, m:], BACK[dt](D0[bi * sd:(bi + 1) * sd]).reshape(n, ldd)[:, m:])
        assert normwise(g[:, :m], w[:, :m]) <= bound, f"batch {bi}"


COMBOS = [("f32", "f32"), ("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32"), ("f32", "bf16")]


@pytest.mark.parametrize("ab,dt", COMBOS)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("bias_mode", [None, "d", "f32"])
def test_matmul_types_layouts_bias(lt, ab, dt, ta, tb, bias_mode):
    run_lt(lt, ab, dt, ta, tb, 192, 136, 72, 1.0, 0.0, bias_mode, False)


@pytest.mark.parametrize("ab,dt", [("f32", "f32"), ("f16", "f16"), ("bf16", "bf16")])
@pytest.mark.parametrize("sep_c", [False, True])
@pytest.mark.parametrize("pmode", [0, 1])
def test_matmul_beta_separate_c_device_scalars(lt, ab, dt, sep_c, pmode):
    run_lt(lt, ab, dt, 0, 1, 256, 192, 128, 0.75, -0.5, "d", sep_c, pmode=pmode)


@pytest.mark.parametrize("ab,dt", [("f32", "f32"), ("f16", "f16"), ("bf16", "bf16")])
def test_matmul_strided_batch_shares_bias(lt, ab, dt):
    run_lt(lt, ab, dt, 1, 0, 96, 80, 64, 1.0, 0.5, "d", True, batch=3)


def test_matmul_large_pipelined_with_bias(lt):
    """a 2048^2 fp16 linear-shaped call (PyTorch addmm with a 1-D bias):
    the pipelined kernel's epilogue adds the bias"""
    import vkblas_amd as vk
    run_lt(lt, "f16", "f16", 1, 0, 2048, 2048, 1024, 1.0, 0.0, "d", False, pads=(8, 8, 8))
    assert vk.last_kernel() in (vk.KERNEL_PIPE256, vk.KERNEL_PIPE128, vk.KERNEL_PIPE128_4)


def test_decode_linear_with_bias(lt):
    """decode shape through hipBLASLt (W (O, K) row-major = column-major K x O
    with transA = T; 4 tokens): the skinny kernels with the bias"""
    import vkblas_amd as vk
    m, n, k = 4096, 4, 2048
    run_lt(lt, "f16", "f16", 1, 0, m, n, k, 1.0, 0.0, "d", False, pads=(0, 0, 0), decode=True)
    assert vk.last_path() == vk.PATH_SKINNY


@pytest.mark.parametrize("what", ["gelu_bias", "relu", "a_scale"])
def test_unsupported_matmuls_are_forwarded(lt, what):
    """activation epilogues and scale pointers go to the real hipBLASLt
    untouched: vkblas_last_path is not changed by the call"""
    import vkblas_amd as vk
    print(f"[case] lt forwarded {what}", flush=True)
    m = n = k = 128
    a = torch.randn(k, m, device="cuda:0").half()
    b = torch.randn(n, k, device="cuda:0").half()
    d = torch.zeros(n, m, device="cuda:0").half()
    bias = torch.randn(m, device="cuda:0").half()
    one = torch.ones(1, device="cuda:0")
    la, lb, ld = lt.layout("f16", m, k, m), lt.layout("f16", k, n, k), lt.layout("f16", m, n, m)
    if what == "gelu_bias":
        desc = lt.desc(0, 0, EPI_GELU_BIAS, bias.data_ptr())
    elif what == "relu":
        desc = lt.desc(0, 0, EPI_RELU)
    else:
        desc = lt.desc(0, 0, scale_ptr=one.data_ptr())
    _mark_skinny(vk)
    ha, hb = ctypes.c_float(1.0), ctypes.c_float(0.0)
    st = lt.ours.hipblasLtMatmul(lt.h, desc, ctypes.addressof(ha), a.data_ptr(), la, b.data_ptr(), lb,
                                 ctypes.addressof(hb), d.data_ptr(), ld, d.data_ptr(), ld, None, None, 0,
                                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert vk.last_path() == vk.PATH_SKINNY
    # the vendor library's answer (any status: the call is its own business)
    del st
    for lay in (la, lb, ld):
        lt.ours.hipblasLtMatrixLayoutDestroy(lay)
    lt.ours.hipblasLtMatmulDescDestroy(desc)


def _sweep_case(i):
    """Seeded random matmul i: types, transposes, shape (decode-shaped or
    general, aligned or ragged), padding, alpha / beta, bias (D's type or
    fp32), C == D or a separate C, strided batch, host or device scalars."""
    r = np.random.default_rng(40000 + i)
    ab, dt = COMBOS[r.integers(len(COMBOS))]
    if r.random() < 0.3:   # decode-shaped: a few columns of D (tokens) against a weight
        m, n, k = int(r.integers(8, 4097)), int(r.integers(1, 17)), int(r.integers(8, 2049))
    else:
        m, n, k = int(r.integers(1, 600)), int(r.integers(1, 600)), int(r.integers(1, 1500))
    if r.random() < 0.6:
        m, k = -(-m // 8) * 8, -(-k // 8) * 8
        pads = tuple(int(8 * r.integers(0, 3)) for _ in range(3))
    else:
        pads = tuple(int(r.integers(0, 9)) for _ in range(3))
    bias_mode = [None, "d", "f32"][r.integers(3)]
    if bias_mode == "f32" and dt == "f32":
        bias_mode = "d"
    return dict(ab=ab, dt=dt, ta=int(r.integers(2)), tb=int(r.integers(2)), m=m, n=n, k=k,
                alpha=float(np.round(r.uniform(-2, 2), 3)),
                beta=0.0 if r.random() < 0.5 else float(np.round(r.uniform(-1.5, 1.5), 3)),
                bias_mode=bias_mode, sep_c=bool(r.random() < 0.3),
                batch=int(r.integers(2, 4)) if r.random() < 0.15 else 1, pmode=int(r.random() < 0.25), pads=pads)


SWEEP = [_sweep_case(i) for i in range(150)]


@pytest.mark.parametrize("c", SWEEP, ids=[f"{i}" for i in range(len(SWEEP))])
def test_matmul_random_sweep(lt, c):
    """150 seeded random matmuls through the interposed hipblasLtMatmul, each
    computed by this library (not forwarded) and checked against the oracle"""
    import vkblas_amd as vk
    # the engine's form of the call (row-major D' = op(B)' op(A)'): which
    # path it takes decides the marker call's path
    dt_ = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    lda = (c["k"] if c["ta"] else c["m"]) + c["pads"][0]
    ldb = (c["n"] if c["tb"] else c["k"]) + c["pads"][1]
    ldd = c["m"] + c["pads"][2]
    pl = vk.plan(dt_[c["ab"]], dt_[c["dt"]], c["tb"], c["ta"], c["n"], c["m"], c["k"], ldb, lda, ldd, c["batch"])
    run_lt(lt, c["ab"], c["dt"], c["ta"], c["tb"], c["m"], c["n"], c["k"], c["alpha"], c["beta"], c["bias_mode"],
           c["sep_c"], batch=c["batch"], pmode=c["pmode"], pads=c["pads"], decode=pl.path == vk.PATH_SKINNY)
