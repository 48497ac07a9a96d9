"""Every GEMM kernel variant against the oracle: tile 64 / 128 / 256, the
generic blocked kernel and the pipelined kernels (256x256, and 128x128 for
16-bit types), the four operand layouts, fp32 and fp16 inputs with fp16 and
fp32 outputs, full tiles and ragged edges, alpha with beta != 0 (C read) and
beta == 0 (C pre-filled with NaN, never read).  Kernels are forced with
vkblas_set_override."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

SHAPES = [(512, 768, 384), (256, 256, 128), (256, 384, 256), (300, 520, 200), (96, 160, 72)]
VARIANTS = [(tile, generic) for tile in (0, 1, 2) for generic in (False, True) if not (generic and tile == 0)]


def rng(seed, n):
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


@pytest.fixture(autouse=True)
def reset_override():
    import vkblas_amd as vk
    yield
    vk.set_override(-1, False)


@pytest.mark.parametrize("tile,generic", VARIANTS, ids=[f"tile{64 << t}{'-generic' if g else ''}" for t, g in VARIANTS])
@pytest.mark.parametrize("dt", ["f32", "f16>f16", "f16>f32"])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SHAPES])
@pytest.mark.parametrize("beta", [-0.5, 0.0])
def test_kernel_variant(tile, generic, dt, op_a, op_b, shape, beta):
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, f32_bound, F16_BOUND
    M, N, K = shape
    print(f"[case] tile={64 << tile} generic={generic} {dt} op={op_a}{op_b} {M}x{N}x{K} beta={beta}", flush=True)
    vk.set_override(tile, generic)
    lda = M if op_a else K
    ldb = K if op_b else N
    ldc = N
    a = rng(M + N + K, lda * (K if op_a else M))
    b = rng(M + 2 * N, ldb * (N if op_b else K))
    c = rng(M + 3 * K, ldc * M)
    if beta == 0.0:
        c[:] = np.nan
    alpha = 0.75
    if dt == "f32":
        ref = c.copy()
        oracle.ref_gemm_f32_rm(op_a, op_b, M, N, K, a, lda, b, ldb, alpha, beta, ref, ldc)
        dA, dB, dC = to_dev(a), to_dev(b), to_dev(c)
        vk.gemm_async(vk.DT_F32, vk.DT_F32, op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb,
                      beta, dC.data_ptr(), ldc, split_k=1)
        assert normwise(to_host(dC), ref) <= f32_bound(K)
        return
    ha, hb = oracle.f2h_rne(a), oracle.f2h_rne(b)
    dA, dB = to_dev(ha), to_dev(hb)
    if dt == "f16>f16":
        hc = oracle.f2h_rne(c)
        ref = hc.copy()
        oracle.ref_gemm_f16_rm(op_a, op_b, M, N, K, ha, lda, hb, ldb, alpha, beta, ref, ldc)
        dC = to_dev(hc)
        vk.gemm_async(vk.DT_F16, vk.DT_F16, op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb,
                      beta, dC.data_ptr(), ldc, split_k=1)
        assert normwise(oracle.h2f(to_host(dC)), oracle.h2f(ref)) <= F16_BOUND
    else:
        ref = c.copy()
        oracle.ref_gemm_f16f32_rm(op_a, op_b, M, N, K, ha, lda, hb, ldb, alpha, beta, ref, ldc)
        dC = to_dev(c)
        vk.gemm_async(vk.DT_F16, vk.DT_F32, op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb,
                      beta, dC.data_ptr(), ldc, split_k=1)
        assert normwise(to_host(dC), ref) <= F16_BOUND


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_pipe128_many_tiles(dt, op_a, op_b):
    """16-bit 128x128 pipelined kernel with more workgroups than CUs (two LDS
    stages, two workgroups per CU): 2304 x 2304 output = 324 tiles; the
    one-workgroup-per-CU grids above take the four-stage form."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND, BF16_BOUND
    M, N, K = 2304, 2304, 384
    print(f"[case] pipe128 many tiles {dt} op={op_a}{op_b}", flush=True)
    vk.set_override(1, False)
    lda = M if op_a else K
    ldb = K if op_b else N
    conv, back, bound = ((oracle.f2h_rne, oracle.h2f, F16_BOUND) if dt == "f16"
                         else (oracle.f2bf_rne, oracle.bf2f, BF16_BOUND))
    vdt = vk.DT_F16 if dt == "f16" else vk.DT_BF16
    ha = conv(rng(11 + op_a, lda * (K if op_a else M)))
    hb = conv(rng(13 + op_b, ldb * (N if op_b else K)))
    dA, dB = to_dev(ha), to_dev(hb)
    dC = torch.full((M * N,), float("nan"), dtype=torch.float16, device="cuda:0")
    vk.gemm_async(vdt, vdt, op_a, op_b, M, N, K, 1.0, dA.data_ptr(), lda, dB.data_ptr(), ldb, 0.0,
                  dC.data_ptr(), N, split_k=1)
    got = to_host(dC)
    rows = oracle.sample_rows(M, 12)
    ref = np.zeros(M * N, np.uint16)
    if dt == "f16":
        oracle.ref_gemm_f16_rm(op_a, op_b, M, N, K, ha, lda, hb, ldb, 1.0, 0.0, ref, N, rows=rows)
    else:
        oracle.ref_gemm_bf16_rm(op_a, op_b, M, N, K, ha, lda, hb, ldb, 1.0, 0.0, ref, N, rows=rows)
    sel = (rows[:, None] * N + np.arange(N)[None, :]).reshape(-1)
    assert np.all(np.isfinite(back(got[sel])))
    assert normwise(back(got[sel]), back(ref[sel])) <= bound
