"""fp32 inputs with a 16-bit result: GemmEx 32F x 32F -> 16F / 16BF (compute
32F), through the engine (every kernel: 64 / 128 / 256 tiles, generic and
pipelined, split-K) and through hipblasGemmEx / rocblas_gemm_ex.

The reference forwarded every mixed Ex combination to the vendor library
(src/vkblas_hipblas.c:428-431); this library computes it: fp32 MFMA
accumulation, alpha * acc + beta * C in fp32, one RNE rounding to the 16-bit
type.  The oracle is the fp32 CPU GEMM (test/test_gemm.c:32-58 arithmetic,
C read as the 16-bit values widened) rounded once to the output type; bars:
fp16 2e-3, bf16 8e-3 normwise.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

SHAPES = [(512, 512, 256), (300, 520, 200), (256, 256, 8192)]


def _u(seed, n):
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


@pytest.fixture(autouse=True)
def reset_override():
    import vkblas_amd as vk
    yield
    vk.set_override(-1, False)


def _ref16(ct, op_a, op_b, M, N, K, a, lda, b, ldb, alpha, beta, c16, ldc):
    """fp32 oracle on the widened C, rounded once to the 16-bit type."""
    to, back = (oracle.f2h_rne, oracle.h2f) if ct == "f16" else (oracle.f2bf_rne, oracle.bf2f)
    c32 = back(c16).astype(np.float32)
    oracle.ref_gemm_f32_rm(op_a, op_b, M, N, K, a, lda, b, ldb, alpha, beta, c32, ldc)
    return to(c32)


@pytest.mark.parametrize("tile", [-1, 0, 1, 2])
@pytest.mark.parametrize("ct", ["f16", "bf16"])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_engine_f32_to_16(tile, ct, op_a, op_b, shape, beta):
    import vkblas_amd as vk
    from gpu_helpers import normwise, F16_BOUND, BF16_BOUND
    M, N, K = shape
    if tile >= 0 and K > 4096:
        pytest.skip("long-K shape runs with the planner (split-K) only")
    print(f"[case] f32>{ct} tile={tile} op={op_a}{op_b} {M}x{N}x{K} beta={beta}", flush=True)
    vk.set_override(tile, False)
    lda = M if op_a else K
    ldb = K if op_b else N
    a = _u(1 + M + op_a, lda * (K if op_a else M))
    b = _u(2 + N + op_b, ldb * (N if op_b else K))
    to, back, tdt, vdt, bound = ((oracle.f2h_rne, oracle.h2f, torch.float16, vk.DT_F16, F16_BOUND) if ct == "f16"
                                 else (oracle.f2bf_rne, oracle.bf2f, torch.bfloat16, vk.DT_BF16, BF16_BOUND))
    c16 = to(_u(3, M * N))
    if beta == 0.0:
        c16 = to(np.full(M * N, np.nan, np.float32))
    ref = _ref16(ct, op_a, op_b, M, N, K, a, lda, b, ldb, 0.75, beta, c16.copy(), N)
    dA, dB = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    dC = torch.from_numpy(c16.view(np.int16)).view(tdt).cuda()
    vk.gemm_async(vk.DT_F32, vdt, op_a, op_b, M, N, K, 0.75, dA.data_ptr(), lda, dB.data_ptr(), ldb, beta,
                  dC.data_ptr(), N)
    torch.cuda.synchronize()
    if K > 4096:
        assert vk.last_path() == vk.PATH_SPLITK
    got = back(dC.cpu().view(torch.int16).numpy().view(np.uint16))
    assert np.all(np.isfinite(got))
    assert normwise(got, back(ref)) <= bound


@pytest.mark.parametrize("ct", ["f16", "bf16"])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
def test_hipblas_gemm_ex_f32_to_16(ct, ta, tb):
    """hipblasGemmEx(32F, 32F, 16F | 16BF, compute 32F), column-major."""
    import vkblas_amd as vk
    from vkblas_amd import hipblas_abi as hb
    from gpu_helpers import Handle, normwise, F16_BOUND, BF16_BOUND
    print(f"[case] hipblasGemmEx f32>{ct} {ta}{tb}", flush=True)
    m, n, k = 192, 320, 128
    lda = (k if ta else m) + 3
    ldb = (n if tb else k) + 1
    ldc = m + 5
    A = _u(11, lda * (m if ta else k))
    B = _u(12, ldb * (k if tb else n))
    to, back, tdt, htype, bound = ((oracle.f2h_rne, oracle.h2f, torch.float16, hb.HIP_R_16F, F16_BOUND)
                                   if ct == "f16" else
                                   (oracle.f2bf_rne, oracle.bf2f, torch.bfloat16, hb.HIP_R_16BF, BF16_BOUND))
    c16 = to(_u(13, ldc * n))
    c32 = back(c16).astype(np.float32)
    oracle.ref_gemm_cm(ta, tb, m, n, k, 1.25, A, lda, B, ldb, -0.5, c32, ldc, 0, threads=0)
    ref = to(c32)
    h = Handle()
    try:
        h.set_stream(torch.cuda.current_stream().cuda_stream)
        dA, dB = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
        dC = torch.from_numpy(c16.view(np.int16)).view(tdt).cuda()
        ops = (hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_T)
        al, be = ctypes.c_float(1.25), ctypes.c_float(-0.5)
        st = h.abi.hipblasGemmEx(h.h, ops[ta], ops[tb], m, n, k, ctypes.byref(al), dA.data_ptr(), hb.HIP_R_32F, lda,
                                 dB.data_ptr(), hb.HIP_R_32F, ldb, ctypes.byref(be), dC.data_ptr(), htype, ldc,
                                 hb.HIPBLAS_COMPUTE_32F, hb.HIPBLAS_GEMM_DEFAULT)
        assert st == hb.HIPBLAS_STATUS_SUCCESS
        torch.cuda.synchronize()
        assert vk.last_path() != vk.PATH_NONE
        got = back(dC.cpu().view(torch.int16).numpy().view(np.uint16)).reshape(n, ldc)[:, :m]
        want = back(ref).reshape(n, ldc)[:, :m]
        assert normwise(got, want) <= bound
        # the padding rows of C (m..ldc) are untouched
        assert np.array_equal(dC.cpu().view(torch.int16).numpy().view(np.uint16).reshape(n, ldc)[:, m:],
                              c16.reshape(n, ldc)[:, m:])
    finally:
        h.close()
