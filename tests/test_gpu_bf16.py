"""bf16 GEMM (reference vkblas_gemm_bf16 / vkblas_gemm_bf16_hipblas,
src/vkblas.h:41-64, src/vkblas.c:3345-3512; hipBLAS routing
src/vkblas_hipblas.c:426-461) against the bf16 CPU oracle: every kernel
variant (tile 64 / 128 / 256, generic and pipelined), the four layouts, bf16
and fp32 outputs, ragged edges, split-K, strided batches, device scalars, the
reference's two C entry points and hipblasGemmEx with 16BF data.
Bars: bf16 result normwise <= 8e-3 (one bf16 ulp), fp32 result <= 2e-3.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

SHAPES = [(512, 768, 384), (256, 256, 128), (300, 520, 200), (96, 160, 72)]
VARIANTS = [(tile, generic) for tile in (0, 1, 2) for generic in (False, True) if not (generic and tile == 0)]


def rng(seed, n, scale=1.0):
    return (np.random.default_rng(seed).uniform(-1.0, 1.0, n) * scale).astype(np.float32)


@pytest.fixture(autouse=True)
def reset_override():
    import vkblas_amd as vk
    yield
    vk.set_override(-1, False)


def _check(got, want, f32_out):
    from gpu_helpers import normwise, F16_BOUND, BF16_BOUND
    if f32_out:
        assert np.all(np.isfinite(got))
        assert normwise(got, want) <= F16_BOUND
    else:
        g, w = oracle.bf2f(got), oracle.bf2f(want)
        assert np.all(np.isfinite(g))
        assert normwise(g, w) <= BF16_BOUND


def _run(op_a, op_b, M, N, K, alpha, beta, f32_out, seed, scale=1.0, split_k=1, lda=None, ldb=None, ldc=None):
    """One engine call on fresh inputs; returns (got, want) host arrays."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    lda = lda or (M if op_a else K)
    ldb = ldb or (K if op_b else N)
    ldc = ldc or N
    ha = oracle.f2bf_rne(rng(seed, lda * (K if op_a else M), scale))
    hb = oracle.f2bf_rne(rng(seed + 1, ldb * (N if op_b else K), scale))
    c = rng(seed + 2, ldc * M)
    hc = c if f32_out else oracle.f2bf_rne(c)
    want = hc.copy()
    if f32_out:
        oracle.ref_gemm_bf16f32_rm(op_a, op_b, M, N, K, ha, lda, hb, ldb, alpha, beta, want, ldc)
    else:
        oracle.ref_gemm_bf16_rm(op_a, op_b, M, N, K, ha, lda, hb, ldb, alpha, beta, want, ldc)
    dA, dB, dC = to_dev(ha), to_dev(hb), to_dev(hc)
    vk.gemm_async(vk.DT_BF16, vk.DT_F32 if f32_out else vk.DT_BF16, op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda,
                  dB.data_ptr(), ldb, beta, dC.data_ptr(), ldc, split_k=split_k,
                  stream=torch.cuda.current_stream().cuda_stream)
    return to_host(dC), want


@pytest.mark.parametrize("tile,generic", VARIANTS, ids=[f"tile{64 << t}{'-generic' if g else ''}" for t, g in VARIANTS])
@pytest.mark.parametrize("out", ["bf16", "f32"])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
@pytest.mark.parametrize("beta", [-0.5, 0.0])
def test_bf16_kernel_variant(tile, generic, out, op_a, op_b, shape, beta):
    import vkblas_amd as vk
    M, N, K = shape
    print(f"[case] bf16 tile={64 << tile} generic={generic} out={out} op={op_a}{op_b} {M}x{N}x{K} beta={beta}",
          flush=True)
    vk.set_override(tile, generic)
    got, want = _run(op_a, op_b, M, N, K, 0.75, beta, out == "f32", M + N + K + op_a)
    _check(got, want, out == "f32")


@pytest.mark.parametrize("op_a,op_b", [(0, 0), (1, 1)])
def test_bf16_range_beyond_fp16(op_a, op_b):
    """Inputs near 2^50 (far outside fp16's range, products near 2^100 within
    fp32's): catches bf16 data read as fp16 anywhere in the path."""
    import vkblas_amd as vk
    print(f"[case] bf16 large range op={op_a}{op_b}", flush=True)
    vk.set_override(2, False)
    got, want = _run(op_a, op_b, 512, 512, 256, 1.0, 0.0, False, 77, scale=2.0 ** 50)
    assert np.abs(oracle.bf2f(want)).max() > 1e29
    _check(got, want, False)


@pytest.mark.parametrize("out", ["bf16", "f32"])
@pytest.mark.parametrize("split", [0, 7])
def test_bf16_splitk(out, split):
    """split 0: the planner's choice for a long K (M = N = 256); 7: forced,
    with ragged slices.  The reduce rounds once to the output type."""
    import vkblas_amd as vk
    M, N, K = 256, 192, 16384 + 40
    print(f"[case] bf16 split-K split={split} out={out}", flush=True)
    p = vk.plan(vk.DT_BF16, vk.DT_F32 if out == "f32" else vk.DT_BF16, 0, 1, M, N, K, K, K, N, split_k=split)
    assert p.path == vk.PATH_SPLITK and p.split > 1
    got, want = _run(0, 1, M, N, K, 1.25, 0.5, out == "f32", 5 + split, split_k=split)
    assert vk.last_path() == vk.PATH_SPLITK
    _check(got, want, out == "f32")


def test_bf16_strided_batched_padded():
    """batch 3 with padded strides and leading dimensions; the padding of C is untouched."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    M, N, K, nb = 200, 136, 96, 3
    lda, ldb, ldc = K + 8, K + 16, N + 5
    sa, sb, sc = lda * M + 40, ldb * N + 24, ldc * M + 7
    print("[case] bf16 strided batched", flush=True)
    A = oracle.f2bf_rne(rng(31, sa * nb))
    B = oracle.f2bf_rne(rng(32, sb * nb))
    C = oracle.f2bf_rne(rng(33, sc * nb))
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    vk.gemm_async(vk.DT_BF16, vk.DT_BF16, 0, 1, M, N, K, 0.5, dA.data_ptr(), lda, dB.data_ptr(), ldb, 1.0,
                  dC.data_ptr(), ldc, batch=nb, stride_a=sa, stride_b=sb, stride_c=sc,
                  stream=torch.cuda.current_stream().cuda_stream)
    got = to_host(dC)
    for i in range(nb):
        want = C[i * sc:(i + 1) * sc].copy()
        oracle.ref_gemm_bf16_rm(0, 1, M, N, K, A[i * sa:], lda, B[i * sb:], ldb, 0.5, 1.0, want, ldc)
        _check(got[i * sc:(i + 1) * sc], want, False)
        pad = np.ones(sc, bool)
        for r in range(M):
            pad[r * ldc: r * ldc + N] = False
        assert np.array_equal(got[i * sc:(i + 1) * sc][pad], C[i * sc:(i + 1) * sc][pad])


def test_bf16_device_scalars():
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    M, N, K = 384, 256, 512
    print("[case] bf16 device scalars", flush=True)
    A = oracle.f2bf_rne(rng(41, M * K))
    B = oracle.f2bf_rne(rng(42, K * N))
    C = oracle.f2bf_rne(rng(43, M * N))
    want = C.copy()
    oracle.ref_gemm_bf16_rm(0, 0, M, N, K, A, K, B, N, -1.5, 0.25, want, N)
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    sc = torch.tensor([-1.5, 0.25], dtype=torch.float32, device="cuda:0")
    vk.gemm_async(vk.DT_BF16, vk.DT_BF16, 0, 0, M, N, K, 0.0, dA.data_ptr(), K, dB.data_ptr(), N, 0.0,
                  dC.data_ptr(), N, scalar_mode=vk.SCALAR_DEV_F32, alpha_dev=sc.data_ptr(),
                  beta_dev=sc.data_ptr() + 4, stream=torch.cuda.current_stream().cuda_stream)
    _check(to_host(dC), want, False)


@pytest.mark.parametrize("entry", ["vkblas_gemm_bf16", "vkblas_gemm_bf16_hipblas"])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_reference_bf16_entry_points(entry, op_a, op_b):
    """The reference's synchronous C entry points: status OK and C written on return."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev
    M, N, K = 333, 270, 130
    lda, ldb, ldc = (M if op_a else K), (K if op_b else N), N
    print(f"[case] {entry} op={op_a}{op_b}", flush=True)
    A = oracle.f2bf_rne(rng(51 + op_a, lda * (K if op_a else M)))
    B = oracle.f2bf_rne(rng(53 + op_b, ldb * (N if op_b else K)))
    C = oracle.f2bf_rne(rng(55, ldc * M))
    want = C.copy()
    oracle.ref_gemm_bf16_rm(op_a, op_b, M, N, K, A, lda, B, ldb, 2.0, -1.0, want, ldc)
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    torch.cuda.synchronize()
    fn = vk.gemm_bf16 if entry == "vkblas_gemm_bf16" else vk.gemm_bf16_hipblas
    st = fn(op_a, op_b, M, N, K, 2.0, dA.data_ptr(), lda, dB.data_ptr(), ldb, -1.0, dC.data_ptr(), ldc)
    assert st == vk.OK
    got = dC.cpu().view(torch.int16).numpy().view(np.uint16)   # no extra synchronisation
    _check(got, want, False)


@pytest.fixture(scope="module")
def handle():
    from gpu_helpers import Handle
    h = Handle()
    yield h
    h.close()


@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_hipblas_gemmex_bf16(handle, ta, tb, out):
    """hipblasGemmEx(16BF, 16BF, {16BF, 32F}, compute 32F), column-major."""
    from gpu_helpers import to_dev, to_host, fbox
    from vkblas_amd import hipblas_abi as hb
    m, n, k = 300, 260, 520
    lda, ldb, ldc = (k if ta else m) + 3, (n if tb else k) + 1, m + 2
    print(f"[case] hipblasGemmEx bf16 {ta}{tb} out={out}", flush=True)
    A = oracle.f2bf_rne(rng(61, lda * (m if ta else k)))
    B = oracle.f2bf_rne(rng(62, ldb * (k if tb else n)))
    C32 = rng(63, ldc * n)
    C = C32 if out == "f32" else oracle.f2bf_rne(C32)
    want = C.copy()
    fn = oracle.ref_gemm_bf16f32_rm if out == "f32" else oracle.ref_gemm_bf16_rm
    fn(tb, ta, n, m, k, B, ldb, A, lda, 0.5, 0.75, want, ldc)     # column-major -> engine
    dA, dB, dC = to_dev(A), to_dev(B), to_dev(C)
    ct = hb.HIP_R_32F if out == "f32" else hb.HIP_R_16BF
    handle.set_stream(torch.cuda.current_stream().cuda_stream)
    st = handle.abi.hipblasGemmEx(handle.h, hb.HIPBLAS_OP_T if ta else hb.HIPBLAS_OP_N,
                                  hb.HIPBLAS_OP_T if tb else hb.HIPBLAS_OP_N, m, n, k, fbox(0.5), dA.data_ptr(),
                                  hb.HIP_R_16BF, lda, dB.data_ptr(), hb.HIP_R_16BF, ldb, fbox(0.75), dC.data_ptr(),
                                  ct, ldc, hb.HIPBLAS_COMPUTE_32F, hb.HIPBLAS_GEMM_DEFAULT)
    assert st == 0
    got = to_host(dC)
    sel = np.concatenate([np.arange(j * ldc, j * ldc + m) for j in range(n)])
    _check(got[sel], want[sel], out == "f32")
    pad = np.ones(got.size, bool)
    pad[sel] = False
    assert np.array_equal(got[pad], C[pad])
