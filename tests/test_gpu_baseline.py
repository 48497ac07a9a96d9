"""Parity at the BASELINE.json configurations (configs 1(ii) and 2-5).

Every case runs this library's kernels through a C-ABI entry point and
compares with the CPU oracle on the same seeded inputs:
  fp32: normwise relative error <= 1e-5 * sqrt(K)       (north star)
  fp16: normwise relative error <= 2e-3                 (north star)
Large shapes compare the oracle's uniformly sampled rows (as test_gemm.c:87
does) -- every column of those rows -- plus size-independent properties
(split-K determinism and split/no-split agreement, batch independence).
"""
import math

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def rng_uniform(seed, n):
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


def rng_normal(seed, n, scale):
    return (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)


# ----------------------------------------------------------------- config 1(ii)

SWEEP_SHAPES = [(1, 1, 1), (3, 5, 7), (64, 1, 64), (127, 129, 65), (256, 256, 256),
                (32, 32, 32), (64, 64, 64), (128, 128, 128), (257, 129, 64), (100, 200, 300),
                (256, 256, 4096), (512, 512, 4096), (512, 640, 4096), (512, 768, 4096), (512, 512, 512),
                (33, 65, 17), (1, 64, 64)]
BIG_SHAPES = [(4096, 4096, 4096), (4096, 1024, 4096), (1024, 4096, 4096)]
AB = [(1.0, 0.0), (1.0, 1.0), (1.0, -0.25), (0.5, 0.0), (0.5, 1.0), (0.5, -0.25)]

SWEEP = [(m, n, k, ta, tb, a, b) for (m, n, k) in SWEEP_SHAPES for ta in (0, 1) for tb in (0, 1) for (a, b) in AB]
SWEEP += [(m, n, k, ta, tb, a, b) for (m, n, k) in BIG_SHAPES for ta in (0, 1) for tb in (0, 1)
          for (a, b) in [(1.0, 0.0), (0.5, -0.25)]]


@pytest.fixture(scope="module")
def handle():
    from gpu_helpers import Handle
    h = Handle()
    yield h
    h.close()


def _run_sgemm_cm(handle, ta, tb, m, n, k, alpha, beta, lda, ldb, ldc, seed, sample):
    from gpu_helpers import to_dev, to_host, fbox
    from vkblas_amd import hipblas_abi as hb
    szA = lda * (m if ta else k)
    szB = ldb * (k if tb else n)
    szC = ldc * n
    hA = rng_uniform(seed, szA)
    hB = rng_uniform(seed + 1, szB)
    hC = rng_uniform(seed + 2, szC)
    hRef = hC.copy()
    oracle.ref_gemm_cm(ta, tb, m, n, k, alpha, hA, lda, hB, ldb, beta, hRef, ldc, sample, threads=0)
    dA, dB, dC = to_dev(hA), to_dev(hB), to_dev(hC)
    ops = (hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_T)
    st = handle.abi.hipblasSgemm(handle.h, ops[ta], ops[tb], m, n, k, fbox(alpha), dA.data_ptr(), lda,
                                 dB.data_ptr(), ldb, fbox(beta), dC.data_ptr(), ldc)
    assert st == 0
    hGot = to_host(dC)
    rows = oracle.sample_rows(m, sample)
    sel = (rows[:, None] + np.arange(n)[None, :] * ldc).reshape(-1)
    return hRef[sel], hGot[sel]


@pytest.mark.parametrize("case", SWEEP, ids=[f"{'NT'[c[3]]}{'NT'[c[4]]} {c[0]}x{c[1]}x{c[2]} a={c[5]} b={c[6]}"
                                             for c in SWEEP])
def test_baseline_sweep_fp32(handle, case):
    """config 1(ii): ld = rows + 3, alpha in {1, .5}, beta in {0, 1, -.25}, U[-1,1)."""
    from gpu_helpers import normwise, f32_bound
    m, n, k, ta, tb, alpha, beta = case
    print(f"[case] sweep {case}", flush=True)
    lda = (k if ta else m) + 3
    ldb = (n if tb else k) + 3
    ldc = m + 3
    seed = (m * 1000003 + n * 10007 + k * 101 + ta * 7 + tb * 3 + int(alpha * 8) * 17 + int(beta * 8 + 8) * 29) % (2**31)
    sample = 12 if m * n * k > 5000000 else 0
    ref, got = _run_sgemm_cm(handle, ta, tb, m, n, k, alpha, beta, lda, ldb, ldc, seed, sample)
    assert np.all(np.isfinite(got))
    assert normwise(got, ref) <= f32_bound(k)


# ----------------------------------------------------------------- config 2

@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_fp32_4096_variants(handle, ta, tb):
    """config 2: M=N=K=4096, ld=4096, alpha=1, beta=0, U[-1,1) (sampled rows)."""
    from gpu_helpers import normwise, f32_bound
    print(f"[case] fp32 4096^3 {'NT'[ta]}{'NT'[tb]}", flush=True)
    ref, got = _run_sgemm_cm(handle, ta, tb, 4096, 4096, 4096, 1.0, 0.0, 4096, 4096, 4096, 2024 + 2 * ta + tb, 12)
    assert normwise(got, ref) <= f32_bound(4096)


# ----------------------------------------------------------------- config 3

def _fp16_inputs(seed, n, K):
    return oracle.f2h_rne(rng_normal(seed, n, 1.0 / math.sqrt(K)))


@pytest.mark.parametrize("size", [2048, 4096, 8192])
@pytest.mark.parametrize("trans", ["NN", "TN"])
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_fp16_gemmex(handle, size, trans, out):
    """config 3: hipblasGemmEx 16F x 16F -> {16F, 32F}, compute 32F, NN and TN."""
    from gpu_helpers import to_dev, to_host, fbox, normwise, F16_BOUND
    from vkblas_amd import hipblas_abi as hb
    M = N = K = size
    print(f"[case] fp16 gemmex {size}^3 {trans} out={out}", flush=True)
    ta = trans[0] == "T"
    hA = _fp16_inputs(10 + size + ta, M * K, K)
    hB = _fp16_inputs(20 + size, K * N, K)
    dA, dB = to_dev(hA), to_dev(hB)
    ct = hb.HIP_R_16F if out == "f16" else hb.HIP_R_32F
    dC = torch.zeros(M * N, dtype=torch.float16 if out == "f16" else torch.float32, device="cuda:0")
    st = handle.abi.hipblasGemmEx(handle.h, hb.HIPBLAS_OP_T if ta else hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_N, M, N, K,
                                  fbox(1.0), dA.data_ptr(), hb.HIP_R_16F, K if ta else M, dB.data_ptr(),
                                  hb.HIP_R_16F, K, fbox(0.0), dC.data_ptr(), ct, M, hb.HIPBLAS_COMPUTE_32F,
                                  hb.HIPBLAS_GEMM_DEFAULT)
    assert st == 0
    hGot = to_host(dC)
    # hipBLAS column-major C(m, n) = engine row-major C'(n, m): engine op_a = N (B, ldb=K: B'[n][k]),
    # engine op_b = transA (A).  Sample 12 engine rows (hipBLAS columns).
    rows = oracle.sample_rows(N, 12)
    if out == "f16":
        ref = np.zeros(M * N, np.uint16)
        oracle.ref_gemm_f16_rm(0, 1 if ta else 0, N, M, K, hB, K, hA, K if ta else M, 1.0, 0.0, ref, M, rows=rows)
        sel = (rows[:, None] * M + np.arange(M)[None, :]).reshape(-1)
        g, r = oracle.h2f(hGot[sel]), oracle.h2f(ref[sel])
    else:
        ref = np.zeros(M * N, np.float32)
        oracle.ref_gemm_f16f32_rm(0, 1 if ta else 0, N, M, K, hB, K, hA, K if ta else M, 1.0, 0.0, ref, M,
                                  rows=rows)
        sel = (rows[:, None] * M + np.arange(M)[None, :]).reshape(-1)
        g, r = hGot[sel], ref[sel]
    assert normwise(g, r) <= F16_BOUND


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_full_output_4096(handle, dtype, ta, tb):
    """configs 2 / 3 at 4096^3 with every element of C compared (the other
    4096^3 cases sample 12 rows, as test_gemm.c:87 does): hipblasSgemm, or
    hipblasGemmEx 16F x 16F -> 16F, in each layout, against the oracle in its
    tiled form (bit for bit the plain oracle: tests/test_oracle.py)."""
    from gpu_helpers import to_dev, to_host, fbox, normwise, f32_bound, F16_BOUND
    from vkblas_amd import hipblas_abi as hb
    n = 4096
    f16 = dtype == "f16"
    print(f"[case] full output {dtype} 4096^3 {'NT'[ta]}{'NT'[tb]}", flush=True)
    if f16:
        hA, hB = _fp16_inputs(70 + 2 * ta + tb, n * n, n), _fp16_inputs(80 + 2 * ta + tb, n * n, n)
    else:
        hA, hB = rng_uniform(90 + 2 * ta + tb, n * n), rng_uniform(100 + 2 * ta + tb, n * n)
    dA, dB = to_dev(hA), to_dev(hB)
    dC = torch.full((n * n,), float("nan"), dtype=torch.float16 if f16 else torch.float32, device="cuda:0")
    ops = (hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_T)
    if f16:
        st = handle.abi.hipblasGemmEx(handle.h, ops[ta], ops[tb], n, n, n, fbox(1.0), dA.data_ptr(), hb.HIP_R_16F,
                                      n, dB.data_ptr(), hb.HIP_R_16F, n, fbox(0.0), dC.data_ptr(), hb.HIP_R_16F, n,
                                      hb.HIPBLAS_COMPUTE_32F, hb.HIPBLAS_GEMM_DEFAULT)
    else:
        st = handle.abi.hipblasSgemm(handle.h, ops[ta], ops[tb], n, n, n, fbox(1.0), dA.data_ptr(), n,
                                     dB.data_ptr(), n, fbox(0.0), dC.data_ptr(), n)
    assert st == 0
    got = to_host(dC)
    # column-major C(m, n) is the engine's row-major C'(n, m) = op_b(B)' op_a(A)'
    ref = np.zeros(n * n, np.uint16 if f16 else np.float32)
    oracle.ref_gemm_tiled_rm(dtype, dtype, tb, ta, n, n, n, hB, n, hA, n, 1.0, 0.0, ref, n)
    if f16:
        got, ref = oracle.h2f(got), oracle.h2f(ref)
    assert np.all(np.isfinite(got))
    assert normwise(got, ref) <= (F16_BOUND if f16 else f32_bound(n))


# ----------------------------------------------------------------- config 4

MV = [(K, O, n) for (K, O) in [(8192, 8192), (4096, 14336), (14336, 4096)] for n in (1, 4, 8, 16)]


@pytest.mark.parametrize("K,O,ntok", MV, ids=[f"K{c[0]}xO{c[1]} n{c[2]}" for c in MV])
@pytest.mark.parametrize("out", ["f16", "f32"])
def test_decode_matvec(handle, K, O, ntok, out):
    """config 4: hipblasGemmEx(T, N, m=O, n=ntok, k=K), W K-contiguous (lda=K)."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, fbox, normwise, F16_BOUND
    from vkblas_amd import hipblas_abi as hb
    print(f"[case] decode K={K} O={O} n={ntok} out={out}", flush=True)
    hW = oracle.f2h_rne(rng_normal(K + O, K * O, 0.02))
    hX = oracle.f2h_rne(rng_normal(K + ntok, K * ntok, 1.0))
    dW, dX = to_dev(hW), to_dev(hX)
    f16 = out == "f16"
    dC = torch.zeros(O * ntok, dtype=torch.float16 if f16 else torch.float32, device="cuda:0")
    st = handle.abi.hipblasGemmEx(handle.h, hb.HIPBLAS_OP_T, hb.HIPBLAS_OP_N, O, ntok, K, fbox(1.0), dW.data_ptr(),
                                  hb.HIP_R_16F, K, dX.data_ptr(), hb.HIP_R_16F, K, fbox(0.0), dC.data_ptr(),
                                  hb.HIP_R_16F if f16 else hb.HIP_R_32F, O, hb.HIPBLAS_COMPUTE_32F,
                                  hb.HIPBLAS_GEMM_DEFAULT)
    assert st == 0
    assert vk.last_path() == vk.PATH_SKINNY
    hGot = to_host(dC)
    # engine: Y[t][o] = sum_k X[t][k] W[o][k]; op_a = N (X, lda=K), op_b = T (W, ldb=K)
    if f16:
        ref = np.zeros(O * ntok, np.uint16)
        oracle.ref_gemm_f16_rm(0, 1, ntok, O, K, hX, K, hW, K, 1.0, 0.0, ref, O)
        g, r = oracle.h2f(hGot), oracle.h2f(ref)
    else:
        ref = np.zeros(O * ntok, np.float32)
        oracle.ref_gemm_f16f32_rm(0, 1, ntok, O, K, hX, K, hW, K, 1.0, 0.0, ref, O)
        g, r = hGot, ref
    assert normwise(g, r) <= F16_BOUND


# ----------------------------------------------------------------- config 5a

@pytest.mark.parametrize("K", [65536, 262144])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("split", [4, 16, 64])
def test_splitk(K, dtype, split):
    """config 5a: M=N=256, tall K, forced split, deterministic two-pass reduce."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, f32_bound, F16_BOUND
    M = N = 256
    print(f"[case] splitk K={K} {dtype} split={split}", flush=True)
    a = rng_uniform(K + 1, M * K)
    b = rng_uniform(K + 2, K * N)
    f16 = dtype == "f16"
    if f16:
        hA, hB = oracle.f2h_rne(a), oracle.f2h_rne(b)
    else:
        hA, hB = a, b
    dA, dB = to_dev(hA), to_dev(hB)
    dt = vk.DT_F16 if f16 else vk.DT_F32
    outs = []
    for rep in range(2):
        dC = torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda:0")
        vk.gemm_async(dt, vk.DT_F32, vk.OP_N, vk.OP_N, M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 0.0,
                      dC.data_ptr(), N, split_k=split)
        assert vk.last_path() == vk.PATH_SPLITK
        outs.append(to_host(dC))
    # bitwise reproducible run to run
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    rows = oracle.sample_rows(M, 12)
    ref = np.zeros(M * N, np.float32)
    if f16:
        oracle.ref_gemm_f16f32_rm(0, 0, M, N, K, hA, K, hB, N, 1.0, 0.0, ref, N, rows=rows)
    else:
        oracle.ref_gemm_f32_rm(0, 0, M, N, K, hA, K, hB, N, 1.0, 0.0, ref, N, rows=rows)
    sel = (rows[:, None] * N + np.arange(N)[None, :]).reshape(-1)
    bound = F16_BOUND if f16 else f32_bound(K)
    assert normwise(outs[0][sel], ref[sel]) <= bound
    # agrees with the unsplit kernel within the same bound
    dC1 = torch.zeros(M * N, dtype=torch.float32, device="cuda:0")
    vk.gemm_async(dt, vk.DT_F32, vk.OP_N, vk.OP_N, M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 0.0,
                  dC1.data_ptr(), N, split_k=1)
    assert normwise(to_host(dC1), outs[0]) <= bound


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("mode", ["auto", "ragged", "ragged128"])
def test_splitk_pipelined(dtype, op_a, op_b, mode):
    """Split-K pass 1 on the pipelined kernel, every layout.  auto: the
    planner's choice at M = N = 256, K = 16384 (128x128 tiles: two-stage for
    fp32, four-stage for 16-bit inputs; alpha = 1, beta = 0, 16-bit output
    for 16-bit inputs); ragged / ragged128: tile forced to 256 / 128, a
    256 x 512 output, split 7 over K = 8448 (the last slice shorter), alpha /
    beta on an fp32 C.  Bitwise reproducible run to run."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, f32_bound, F16_BOUND, BF16_BOUND
    auto = mode == "auto"
    M, N, K = (256, 256, 16384) if auto else (256, 512, 8448)
    alpha, beta = (1.0, 0.0) if auto else (0.75, -0.5)
    print(f"[case] splitk pipelined {dtype} op={op_a}{op_b} {mode}", flush=True)
    lda = M if op_a else K
    ldb = K if op_b else N
    a = rng_uniform(300 + op_a, M * K)
    b = rng_uniform(302 + op_b, K * N)
    c = rng_uniform(304, M * N)
    dt = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}[dtype]
    conv = {"f32": lambda x: x, "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}[dtype]
    hA, hB = conv(a), conv(b)
    out16 = auto and dtype != "f32"
    ct = dt if out16 else vk.DT_F32
    hC = conv(c) if out16 else c
    if not auto:
        vk.set_override(1 if mode == "ragged128" else 2, False)
    try:
        pl = vk.plan(dt, ct, op_a, op_b, M, N, K, lda, ldb, N, split_k=0 if auto else 7)
        # the planner: 128x128 tiles
        tile = 2 if mode == "ragged" else 1
        assert pl.path == vk.PATH_SPLITK and pl.tile == tile
        step2 = 64 if dtype == "f32" else 128
        assert pl.k_per_split % step2 == 0 and (K - (pl.split - 1) * pl.k_per_split) % step2 == 0
        if auto:
            edge = 64 << tile
            assert pl.split * (M // edge) * (N // edge) >= 64
        else:
            assert K - (pl.split - 1) * pl.k_per_split < pl.k_per_split
        dA, dB = to_dev(hA), to_dev(hB)
        outs = []
        for _ in range(2):
            dC = to_dev(hC)
            vk.gemm_async(dt, ct, op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb, beta,
                          dC.data_ptr(), N, split_k=0 if auto else 7)
            assert vk.last_path() == vk.PATH_SPLITK
            # pipelined pass 1: 256x256, or 128x128 (one workgroup per CU or
            # fewer: four stages for 16-bit inputs, two for fp32)
            kern = vk.KERNEL_PIPE256 if tile == 2 else (vk.KERNEL_PIPE128 if dtype == "f32" else vk.KERNEL_PIPE128_4)
            assert vk.last_kernel() == kern, vk.last_kernel()
            outs.append(to_host(dC))
    finally:
        vk.set_override(-1, False)
    assert np.array_equal(outs[0], outs[1])
    rows = oracle.sample_rows(M, 12)
    sel = (rows[:, None] * N + np.arange(N)[None, :]).reshape(-1)
    ref = hC.copy()
    if dtype == "f32":
        oracle.ref_gemm_f32_rm(op_a, op_b, M, N, K, hA, lda, hB, ldb, alpha, beta, ref, N, rows=rows)
        assert normwise(outs[0][sel], ref[sel]) <= f32_bound(K)
    elif dtype == "f16":
        if out16:
            oracle.ref_gemm_f16_rm(op_a, op_b, M, N, K, hA, lda, hB, ldb, alpha, beta, ref, N, rows=rows)
            assert normwise(oracle.h2f(outs[0][sel]), oracle.h2f(ref[sel])) <= F16_BOUND
        else:
            oracle.ref_gemm_f16f32_rm(op_a, op_b, M, N, K, hA, lda, hB, ldb, alpha, beta, ref, N, rows=rows)
            assert normwise(outs[0][sel], ref[sel]) <= F16_BOUND
    else:
        if out16:
            oracle.ref_gemm_bf16_rm(op_a, op_b, M, N, K, hA, lda, hB, ldb, alpha, beta, ref, N, rows=rows)
            assert normwise(oracle.bf2f(outs[0][sel]), oracle.bf2f(ref[sel])) <= BF16_BOUND
        else:
            oracle.ref_gemm_bf16f32_rm(op_a, op_b, M, N, K, hA, lda, hB, ldb, alpha, beta, ref, N, rows=rows)
            assert normwise(outs[0][sel], ref[sel]) <= F16_BOUND


@pytest.mark.parametrize("trans", ["NN", "TT"])
def test_splitk_fp16_out_alpha_beta(trans):
    """split-K pass 2 applies alpha/beta once and rounds once to fp16."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND
    M, N, K = 96, 160, 20000
    op = vk.OP_T if trans == "TT" else vk.OP_N
    hA = oracle.f2h_rne(rng_uniform(5, M * K))
    hB = oracle.f2h_rne(rng_uniform(6, K * N))
    hC = oracle.f2h_rne(rng_uniform(7, M * N))
    lda = M if op else K
    ldb = K if op else N
    ref = hC.copy()
    oracle.ref_gemm_f16_rm(op, op, M, N, K, hA, lda, hB, ldb, 0.5, -0.25, ref, N)
    dA, dB, dC = to_dev(hA), to_dev(hB), to_dev(hC)
    vk.gemm_async(vk.DT_F16, vk.DT_F16, op, op, M, N, K, 0.5, dA.data_ptr(), lda, dB.data_ptr(), ldb, -0.25,
                  dC.data_ptr(), N, split_k=8)
    assert vk.last_path() == vk.PATH_SPLITK
    assert normwise(oracle.h2f(to_host(dC)), oracle.h2f(ref)) <= F16_BOUND


def test_splitk_workspace_per_stream():
    """Split-K partials live in a workspace kept per stream.  Calls queued on
    two streams with no synchronisation in between, each stream's later calls
    needing more partials than its earlier ones (the workspace grows while
    earlier calls are still queued), every call made twice: each result
    matches the oracle and the two runs of a call are bitwise equal."""
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, f32_bound
    print("[case] splitk workspace, two streams", flush=True)
    cases = [(64, 64, 8192, 8), (128, 128, 8192, 16), (256, 256, 8192, 32), (128, 256, 16384, 64)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    jobs = []
    for si in range(2):
        for ci, (M, N, K, split) in enumerate(cases):
            a = rng_uniform(500 + 10 * si + ci, M * K)
            b = rng_uniform(600 + 10 * si + ci, K * N)
            outs = [torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda:0") for _ in range(2)]
            jobs.append((streams[si], M, N, K, split, a, b, to_dev(a), to_dev(b), outs))
    torch.cuda.synchronize()
    for rep in range(2):
        for ci in range(len(cases)):
            for si in range(2):
                st, M, N, K, split, _, _, dA, dB, outs = jobs[si * len(cases) + ci]
                vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, vk.OP_N, M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(),
                              N, 0.0, outs[rep].data_ptr(), N, split_k=split, stream=st.cuda_stream)
                assert vk.last_path() == vk.PATH_SPLITK
    torch.cuda.synchronize()
    for st, M, N, K, split, a, b, _, _, outs in jobs:
        h0, h1 = to_host(outs[0]), to_host(outs[1])
        assert np.array_equal(h0.view(np.uint32), h1.view(np.uint32))
        rows = oracle.sample_rows(M, 12)
        ref = np.zeros(M * N, np.float32)
        oracle.ref_gemm_f32_rm(0, 0, M, N, K, a, K, b, N, 1.0, 0.0, ref, N, rows=rows)
        sel = (rows[:, None] * N + np.arange(N)[None, :]).reshape(-1)
        assert normwise(h0[sel], ref[sel]) <= f32_bound(K)


def test_splitk_workspace_threads():
    """Host threads issuing split-K calls at once, each on its own stream
    (the workspace table is shared, each stream's workspace is not): every
    result equals the same call made alone, bit for bit."""
    import threading
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    print("[case] splitk workspace, four threads", flush=True)
    M, N, K = 128, 128, 16384
    nthreads, calls = 4, 6
    a = [to_dev(rng_uniform(700 + t, M * K)) for t in range(nthreads)]
    b = [to_dev(rng_uniform(710 + t, K * N)) for t in range(nthreads)]
    splits = (4, 16, 64)
    alone = {}
    for t in range(nthreads):
        for sp in splits:
            c = torch.empty(M * N, dtype=torch.float32, device="cuda:0")
            vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, vk.OP_N, M, N, K, 1.0, a[t].data_ptr(), K, b[t].data_ptr(),
                          N, 0.0, c.data_ptr(), N, split_k=sp)
            alone[t, sp] = to_host(c)
    outs = [[torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda:0") for _ in range(calls)]
            for _ in range(nthreads)]
    streams = [torch.cuda.Stream() for _ in range(nthreads)]
    torch.cuda.synchronize()
    errors = []

    def worker(t):
        try:
            for i in range(calls):
                # splits 4, 16, 64, 4, ...: the stream's workspace grows while
                # its earlier calls are still queued
                vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, vk.OP_N, M, N, K, 1.0, a[t].data_ptr(), K,
                              b[t].data_ptr(), N, 0.0, outs[t][i].data_ptr(), N, split_k=splits[i % 3],
                              stream=streams[t].cuda_stream)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(nthreads)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors
    torch.cuda.synchronize()
    for t in range(nthreads):
        for i in range(calls):
            assert np.array_equal(to_host(outs[t][i]).view(np.uint32), alone[t, splits[i % 3]].view(np.uint32))


# ----------------------------------------------------------------- config 5b

def test_strided_batched_64x512(handle):
    """config 5b: hipblasSgemmStridedBatched NN, batch 64 of 512^3."""
    from gpu_helpers import to_dev, to_host, fbox, normwise, f32_bound
    from vkblas_amd import hipblas_abi as hb
    nb, n = 64, 512
    s = n * n
    hA = rng_uniform(51, nb * s)
    hB = rng_uniform(52, nb * s)
    dA, dB = to_dev(hA), to_dev(hB)
    dC = torch.zeros(nb * s, dtype=torch.float32, device="cuda:0")
    st = handle.abi.hipblasSgemmStridedBatched(handle.h, hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_N, n, n, n, fbox(1.0),
                                               dA.data_ptr(), n, s, dB.data_ptr(), n, s, fbox(0.0), dC.data_ptr(),
                                               n, s, nb)
    assert st == 0
    hGot = to_host(dC)
    rows = oracle.sample_rows(n, 12)
    for b in range(nb):   # every batch, the same 12 sampled rows of each
        ref = np.zeros(s, np.float32)
        oracle.ref_gemm_cm(0, 0, n, n, n, 1.0, np.ascontiguousarray(hA[b * s:(b + 1) * s]), n,
                           np.ascontiguousarray(hB[b * s:(b + 1) * s]), n, 0.0, ref, n, 12, threads=0)
        sel = (rows[:, None] + np.arange(n)[None, :] * n).reshape(-1)
        assert normwise(hGot[b * s:][sel], ref[sel]) <= f32_bound(n)
