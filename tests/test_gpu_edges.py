"""Edge semantics of the boundary (reference src/vkblas.h:21-26 and
src/vkblas_hipblas.c), each against the oracle or a closed form."""
import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def rng(seed, n):
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("shape", [(64, 64, 64), (256, 256, 128), (33, 65, 17)])
def test_beta_zero_never_reads_c(dtype, shape):
    """beta == 0: C pre-filled with NaN must not leak (src/vkblas.h:26)."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    M, N, K = shape
    f16 = dtype == "f16"
    a, b = rng(1, M * K), rng(2, K * N)
    hA, hB = (oracle.f2h_rne(a), oracle.f2h_rne(b)) if f16 else (a, b)
    dC = torch.full((M * N,), float("nan"), dtype=torch.float16 if f16 else torch.float32, device="cuda:0")
    fn = vk.gemm_f16 if f16 else vk.gemm_f32
    assert fn(0, 0, M, N, K, 1.0, to_dev(hA).data_ptr(), K, to_dev(hB).data_ptr(), N, 0.0, dC.data_ptr(), N) == vk.OK
    got = to_host(dC)
    got = oracle.h2f(got) if f16 else got
    assert np.all(np.isfinite(got))


def test_alpha_zero_scales_c():
    """alpha == 0: C = beta * C exactly (closed form)."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    M, N, K = 128, 96, 64
    hC = rng(3, M * N)
    dC = to_dev(hC)
    assert vk.gemm_f32(0, 1, M, N, K, 0.0, to_dev(rng(4, M * K)).data_ptr(), K, to_dev(rng(5, N * K)).data_ptr(), K,
                       0.5, dC.data_ptr(), N) == vk.OK
    assert np.array_equal(to_host(dC), (np.float32(0.5) * hC).astype(np.float32))


@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_identity_copies_b(op_a, op_b):
    """A = I: C = B exactly for every variant (closed form)."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    n = 160
    hA = np.eye(n, dtype=np.float32).reshape(-1)
    Bm = rng(6, n * n).reshape(n, n)          # logical B_eff[k][n]
    hB = (Bm.T if op_b else Bm).copy().reshape(-1)
    dC = torch.zeros(n * n, dtype=torch.float32, device="cuda:0")
    assert vk.gemm_f32(op_a, op_b, n, n, n, 1.0, to_dev(hA).data_ptr(), n, to_dev(hB).data_ptr(), n, 0.0,
                       dC.data_ptr(), n) == vk.OK
    assert np.array_equal(to_host(dC).reshape(n, n), Bm)


def test_small_integers_exact():
    """Small-integer data sum exactly in fp32 (cf. test/test_cache.c:10-22)."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    M, N, K = 100, 50, 200
    A = (np.arange(M * K) % 3).astype(np.float32).reshape(M, K)
    B = ((np.arange(K * N) % 4) + 1.0).astype(np.float32).reshape(K, N)
    dC = torch.zeros(M * N, dtype=torch.float32, device="cuda:0")
    assert vk.gemm_f32(0, 0, M, N, K, 1.0, to_dev(A.reshape(-1)).data_ptr(), K, to_dev(B.reshape(-1)).data_ptr(), N,
                       0.0, dC.data_ptr(), N) == vk.OK
    exact = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    assert np.array_equal(to_host(dC).reshape(M, N), exact)


@pytest.mark.parametrize("k", [1, 2, 3])
def test_tiny_k_outer_product(k):
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    M, N = 70, 90
    a, b = rng(7, M * k), rng(8, k * N)
    dC = torch.zeros(M * N, dtype=torch.float32, device="cuda:0")
    assert vk.gemm_f32(0, 0, M, N, k, 1.0, to_dev(a).data_ptr(), k, to_dev(b).data_ptr(), N, 0.0, dC.data_ptr(),
                       N) == vk.OK
    ref = np.zeros(M * N, np.float32)
    oracle.ref_gemm_f32_rm(0, 0, M, N, k, a, k, b, N, 1.0, 0.0, ref, N)
    assert np.allclose(to_host(dC), ref, rtol=1e-6, atol=1e-6)


def test_pointer_mode_device_sgemm():
    """HIPBLAS_POINTER_MODE_DEVICE: alpha/beta read by the kernel from device memory."""
    from gpu_helpers import Handle, to_dev, to_host, normwise, f32_bound
    from vkblas_amd import hipblas_abi as hb
    m, n, k = 200, 130, 300
    hA, hB, hC = rng(9, m * k), rng(10, k * n), rng(11, m * n)
    ref = hC.copy()
    oracle.ref_gemm_cm(0, 0, m, n, k, 0.75, hA, m, hB, k, -0.5, ref, m, 0)
    dA, dB, dC = to_dev(hA), to_dev(hB), to_dev(hC)
    scal = torch.tensor([0.75, -0.5], dtype=torch.float32, device="cuda:0")
    h = Handle()
    try:
        h.set_pointer_mode(hb.HIPBLAS_POINTER_MODE_DEVICE)
        st = h.abi.hipblasSgemm(h.h, hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_N, m, n, k, scal.data_ptr(), dA.data_ptr(), m,
                                dB.data_ptr(), k, scal.data_ptr() + 4, dC.data_ptr(), m)
        assert st == 0
        got = to_host(dC)
    finally:
        h.close()
    assert normwise(got, ref) <= f32_bound(k)


def test_hgemm_half_scalars_and_stream():
    """hipblasHgemm: hipblasHalf alpha/beta, launched on the handle's stream."""
    from gpu_helpers import Handle, to_dev, to_host, hbox, normwise, F16_BOUND
    from vkblas_amd import hipblas_abi as hb
    m, n, k = 192, 136, 72
    hA, hB, hC = oracle.f2h_rne(rng(12, m * k)), oracle.f2h_rne(rng(13, k * n)), oracle.f2h_rne(rng(14, m * n))
    # column-major hipBLAS NT: C(m,n) = A(m,k) B(n,k)^T ; engine: op_a = T (B), op_b = N (A)
    ref = hC.copy()
    oracle.ref_gemm_f16_rm(1, 0, n, m, k, hB, n, hA, m, 2.0, 0.5, ref, m)
    s = torch.cuda.Stream()
    dA, dB, dC = to_dev(hA), to_dev(hB), to_dev(hC)
    torch.cuda.synchronize()
    h = Handle()
    try:
        h.set_stream(s.cuda_stream)
        st = h.abi.hipblasHgemm(h.h, hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_T, m, n, k, hbox(2.0), dA.data_ptr(), m,
                                dB.data_ptr(), n, hbox(0.5), dC.data_ptr(), m)
        assert st == 0
        s.synchronize()
        got = to_host(dC)
    finally:
        h.close()
    assert normwise(oracle.h2f(got), oracle.h2f(ref)) <= F16_BOUND


@pytest.mark.parametrize("ldc_pad", [0, 1, 3])
def test_fp16_odd_ld_and_n(ldc_pad):
    """fp16 with odd N / ldc (the reference needed a conversion fallback)."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND
    M, N, K = 77, 131, 45
    lda, ldb, ldc = K + 1, N + 2, N + ldc_pad
    hA = oracle.f2h_rne(rng(15, M * lda))
    hB = oracle.f2h_rne(rng(16, K * ldb))
    hC = oracle.f2h_rne(rng(17, M * ldc))
    ref = hC.copy()
    oracle.ref_gemm_f16_rm(0, 0, M, N, K, hA, lda, hB, ldb, 1.0, 1.0, ref, ldc)
    dC = to_dev(hC)
    assert vk.gemm_f16(0, 0, M, N, K, 1.0, to_dev(hA).data_ptr(), lda, to_dev(hB).data_ptr(), ldb, 1.0,
                       dC.data_ptr(), ldc) == vk.OK
    assert normwise(oracle.h2f(to_host(dC)), oracle.h2f(ref)) <= F16_BOUND


def test_negative_batch_stride():
    """int64 strides may be negative: batch b uses base + b*stride."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, f32_bound
    M, N, K, nb = 64, 48, 32, 3
    sa = M * K
    hA = rng(18, nb * sa)
    hB = rng(19, K * N)
    dA = to_dev(hA)
    dC = torch.zeros(nb * M * N, dtype=torch.float32, device="cuda:0")
    last = dA.data_ptr() + (nb - 1) * sa * 4
    assert vk.gemm_f32(0, 0, M, N, K, 1.0, last, K, to_dev(hB).data_ptr(), N, 0.0, dC.data_ptr(), N, nb, -sa, 0,
                       M * N) == vk.OK
    got = to_host(dC)
    for b in range(nb):
        ref = np.zeros(M * N, np.float32)
        src = np.ascontiguousarray(hA[(nb - 1 - b) * sa:(nb - b) * sa])
        oracle.ref_gemm_f32_rm(0, 0, M, N, K, src, K, hB, N, 1.0, 0.0, ref, N)
        assert normwise(got[b * M * N:(b + 1) * M * N], ref) <= f32_bound(K)


def test_engine_rejects_bad_params():
    import vkblas_amd as vk
    x = torch.zeros(64, device="cuda:0")
    p = x.data_ptr()
    assert vk.gemm_f32(0, 0, 0, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4) == vk.ERR_PARAM
    assert vk.gemm_f32(0, 0, 4, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4, 0) == vk.ERR_PARAM
    assert vk.gemm_f32(0, 0, 4, 4, 8, 1.0, p, 0, p, 4, 0.0, p, 4) == vk.ERR_PARAM   # lda == 0
    assert vk.gemm_bf16(0, 0, 0, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4) == vk.ERR_PARAM
    assert vk.gemm_bf16(0, 0, 4, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4, 0) == vk.ERR_PARAM
    assert vk.gemm_bf16_hipblas(0, 0, 4, 4, 4, 1.0, p, 0, p, 4, 0.0, p, 4) == vk.ERR_PARAM


def test_hipblas_zero_size_forwards():
    """m == 0 goes to the real hipBLAS (quick return SUCCESS, C untouched)."""
    from gpu_helpers import Handle, fbox
    from vkblas_amd import hipblas_abi as hb
    x = torch.ones(16, device="cuda:0")
    h = Handle()
    try:
        st = h.abi.hipblasSgemm(h.h, hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_N, 0, 4, 4, fbox(1.0), x.data_ptr(), 1,
                                x.data_ptr(), 4, fbox(0.0), x.data_ptr(), 1)
    finally:
        h.close()
    assert st == hb.HIPBLAS_STATUS_SUCCESS
    torch.cuda.synchronize()
    assert torch.all(x == 1)
