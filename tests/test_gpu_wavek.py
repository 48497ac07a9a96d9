"""Split-K pass 1 on 32x32 / 64x64 tiles (gemm_wavek_kernel).

A caller's split that 128x128 tiles cannot spread over the chip runs pass 1
on 64x64 tiles when they give at least 224 workgroups, else on 32x32 tiles;
each of a workgroup's four waves takes a quarter of the slice's K steps and
the four sums are added in wave order.  Cases: every layout (engine op_a /
op_b), fp32 / fp16 / bf16 inputs with fp32 results, K slices that do not
divide evenly over the waves and a last slice shorter than the others, the
BASELINE configs[4] splits 4 and 16 at M = N = 256, alpha / beta / a separate
C_in and a bias applied once by the reduce.  Checked against the CPU oracle
over the whole output (normwise), bitwise run-to-run
reproducibility, and the kernel that ran."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

CONV = {"f32": lambda x: x, "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}


def _u(seed, n):
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


def _dev(a, dt):
    a = np.ascontiguousarray(a)
    if dt == "f32":
        return torch.from_numpy(a).to("cuda:0")
    t = torch.from_numpy(a.view(np.int16))
    return t.view(torch.float16 if dt == "f16" else torch.bfloat16).to("cuda:0")


def _ref(dt, op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, ldc):
    if dt == "f32":
        oracle.ref_gemm_f32_rm(op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, ldc)
    elif dt == "f16":
        oracle.ref_gemm_f16f32_rm(op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, ldc)
    else:
        oracle.ref_gemm_bf16f32_rm(op_a, op_b, M, N, K, A, lda, B, ldb, alpha, beta, C, ldc)


# (M, N, K, split, expected tile code): 64x64 tiles (0) where they give >=
# 224 workgroups; else 64x64 tiles with each K slice over four workgroups (4)
# where that gives 224 and the slices hold at least 16 K steps; else 32x32 (3)
SHAPES = [(256, 256, 8256, 4, 4), (256, 256, 8192, 16, 0), (64, 128, 3008, 3, 3), (192, 96, 4096, 5, 3),
          (512, 256, 2048, 8, 0), (256, 256, 1024, 4, 3), (128, 256, 16384, 9, 4)]


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}s{s}" for m, n, k, s, _ in SHAPES])
def test_wavek_layouts(dt, op_a, op_b, shape):
    import vkblas_amd as vk
    from gpu_helpers import to_host, normwise, f32_bound, F16_BOUND
    M, N, K, split, tt = shape
    print(f"[case] wavek {dt} op={op_a}{op_b} {M}x{N}x{K} split={split}", flush=True)
    lda = M if op_a else K
    ldb = K if op_b else N
    hA = CONV[dt](_u(M + K + op_a, M * K))
    hB = CONV[dt](_u(N + K + 2 * op_b + 7, K * N))
    code = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}[dt]
    pl = vk.plan(code, vk.DT_F32, op_a, op_b, M, N, K, lda, ldb, N, split_k=split)
    assert pl.path == vk.PATH_SPLITK and pl.split == split
    assert pl.tile == tt, (pl.tile, tt)
    dA, dB = _dev(hA, dt), _dev(hB, dt)
    outs = []
    for _ in range(2):
        dC = torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda:0")
        vk.gemm_async(code, vk.DT_F32, op_a, op_b, M, N, K, 1.0, dA.data_ptr(), lda, dB.data_ptr(), ldb, 0.0,
                      dC.data_ptr(), N, split_k=split)
        assert vk.last_path() == vk.PATH_SPLITK
        assert vk.last_kernel() == vk.KERNEL_WAVEK, vk.last_kernel()
        outs.append(to_host(dC))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    ref = np.zeros(M * N, np.float32)
    _ref(dt, op_a, op_b, M, N, K, hA, lda, hB, ldb, 1.0, 0.0, ref, N)
    bound = f32_bound(K) if dt == "f32" else F16_BOUND
    assert normwise(outs[0], ref) <= bound


@pytest.mark.parametrize("dt", ["f32", "f16"])
@pytest.mark.parametrize("split", [4, 16])
def test_wavek_epilogue(dt, split):
    """alpha, beta, a separate C_in and a bias, applied once by the reduce
    (pass 1 writes raw sums); C_in is not written."""
    import vkblas_amd as vk
    from gpu_helpers import to_host, normwise, f32_bound, F16_BOUND
    M = N = 256
    K = 4096 + 64 * split
    print(f"[case] wavek epilogue {dt} split={split}", flush=True)
    hA = CONV[dt](_u(11, M * K))
    hB = CONV[dt](_u(12, K * N))
    cin = _u(13, M * N)
    bias = _u(14, N)
    want = np.zeros(M * N, np.float32)
    oracle.ref_gemm_epi_rm(dt, "f32", 0, 0, M, N, K, hA, K, hB, N, 0.75, -0.5, cin, N, want, N, bias=bias)
    code = {"f32": vk.DT_F32, "f16": vk.DT_F16}[dt]
    dA, dB = _dev(hA, dt), _dev(hB, dt)
    dCin = torch.from_numpy(cin).to("cuda:0")
    dBias = torch.from_numpy(bias).to("cuda:0")
    dD = torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda:0")
    vk.gemm_ex_async(code, vk.DT_F32, 0, 0, M, N, K, 0.75, dA.data_ptr(), K, dB.data_ptr(), N, -0.5,
                     dD.data_ptr(), N, split_k=split, c_in=dCin.data_ptr(), ldc_in=N, bias=dBias.data_ptr(),
                     bias_type=vk.DT_F32)
    assert vk.last_kernel() == vk.KERNEL_WAVEK
    assert np.array_equal(to_host(dCin), cin)
    bound = f32_bound(K) if dt == "f32" else F16_BOUND
    assert normwise(to_host(dD), want) <= bound


def test_wavek_divided_slices_repeat():
    """Each K slice over four workgroups (the last to arrive adds the four
    sums): calls of three shapes interleaved on one stream, each repeated,
    give the first call's result bit for bit (the arrival counters stay in
    step across calls and shapes), and the oracle's within the bound."""
    import vkblas_amd as vk
    from gpu_helpers import to_host, normwise, f32_bound
    print("[case] wavek divided slices, repeated", flush=True)
    cases = [(256, 256, 16384, 4), (128, 256, 16384, 9), (256, 256, 8256, 5)]
    data = []
    for i, (M, N, K, split) in enumerate(cases):
        pl = vk.plan(vk.DT_F32, vk.DT_F32, 0, 0, M, N, K, K, N, N, split_k=split)
        assert (pl.path, pl.split, pl.tile) == (vk.PATH_SPLITK, split, 4), (M, N, K, split, pl.tile)
        hA, hB = _u(50 + i, M * K), _u(60 + i, K * N)
        data.append((hA, hB, torch.from_numpy(hA).to("cuda:0"), torch.from_numpy(hB).to("cuda:0")))
    first = {}
    for rep in range(3):
        for i, (M, N, K, split) in enumerate(cases):
            _, _, dA, dB = data[i]
            dC = torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda:0")
            vk.gemm_async(vk.DT_F32, vk.DT_F32, 0, 0, M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 0.0,
                          dC.data_ptr(), N, split_k=split)
            assert vk.last_kernel() == vk.KERNEL_WAVEK
            got = to_host(dC)
            if rep == 0:
                first[i] = got
            else:
                assert np.array_equal(got.view(np.uint32), first[i].view(np.uint32)), (rep, cases[i])
    for i, (M, N, K, split) in enumerate(cases):
        hA, hB, _, _ = data[i]
        ref = np.zeros(M * N, np.float32)
        oracle.ref_gemm_f32_rm(0, 0, M, N, K, hA, K, hB, N, 1.0, 0.0, ref, N)
        assert normwise(first[i], ref) <= f32_bound(K), cases[i]
