"""The fp32 skinny kernels (engine op_a = N, fp32 output), the path of the
reference's fp32 matvec (src/vkblas.c:2100-2143, 2501-2607;
shaders/matvec_f32_tmpl.comp:23-74, TB = 0 and TB = 1):

  op_b = T: W stored N x K (each output's K weights contiguous), up to 64
            activation rows: the staged MFMA skinny kernel with 16-byte
            fragments of 4 floats (M <= 16), the staged decode kernel with
            a K split over the grid (17 <= M <= 64);
  op_b = N: W stored K x N (N-contiguous rows), up to 64 rows: the K x N MFMA kernel, with
            a K split over the grid for long K (fp32 partials + the
            fixed-order reduce).

Ragged K (not a multiple of the kernels' 64-float and 16-row K steps), K
smaller than one step, N not a multiple of the workgroup's columns, padded
leading dimensions whose padding holds NaN (it must never reach C), padded
C columns that must stay untouched, beta != 0, a separate C input and a bias
(vkblas_gemm_ex_async), device-memory scalars, determinism of the split.
The oracle is the fp32 CPU restatement of the engine contract; the bar is
the north-star fp32 bound, normwise <= 1e-5 sqrt(K).
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

SENT = np.float32(-7.25)   # value of C's padding columns, checked afterwards

# (M, N, K, pad_a, pad_b, pad_c, beta): lda = K + pad_a and ldb = K + pad_b
# (N x K) or N + pad_b (K x N) are multiples of 4 (lda may be anything for M = 1)
CASES_T = []
for M in (1, 2, 3, 4, 5, 8, 9, 16):
    for (N, K) in ((1, 4), (7, 252), (100, 260), (1000, 1028), (300, 4100), (64, 8192)):
        CASES_T.append((M, N, K, 0, 0, 0, 0.0))
CASES_T += [
    (1, 300, 1001, 3, 7, 0, 0.0),
    (2, 257, 4099, 1, 5, 4, 0.5),
    (3, 64, 13, 3, 3, 1, 0.0),
    (4, 129, 2051, 1, 1, 0, -0.5),
    (8, 8192, 1000, 0, 4, 0, 0.0),       # 512 workgroups, 16 K steps: two waves each
    (12, 8200, 1032, 4, 4, 3, 0.25),     # two weight tiles per workgroup, ragged last one
    (16, 8192, 520, 0, 0, 0, 0.5),
    (10, 8240, 3000, 4, 0, 0, 0.5),      # two tiles, two waves, three stages over 46 K steps
    (16, 64, 13, 3, 3, 2, -0.5),
    # 17-64 rows: the decode kernel, 64-float K steps, ragged last step
    (17, 1000, 1028, 0, 0, 0, 0.0),
    (20, 64, 13, 3, 3, 2, -0.5),         # no full step: the checked tail only
    (24, 300, 4100, 4, 4, 1, 0.5),       # K split, the last slice ending in a partial step
    (32, 4096, 4096, 0, 0, 0, 0.0),      # two weight tiles per wave, K split
    (33, 257, 2051, 1, 1, 0, -0.5),      # three activation tiles, the last one row
    (48, 8192, 1000, 0, 4, 0, 0.0),
    (64, 4096, 4100, 4, 0, 3, 0.25),
    (64, 129, 64, 0, 0, 0, 0.0),         # one full step, unsplit
]

CASES_N = []
for M in (1, 2, 4, 5, 8, 16):
    for (N, K) in ((4, 1), (8, 15), (100, 260), (1000, 1028), (4096, 4100), (256, 8192), (8192, 1000)):
        CASES_N.append((M, N, K, -K % 4, 0, 0, 0.0))   # lda a multiple of 4
CASES_N += [
    (1, 300, 1001, 5, 4, 0, 0.0),
    (2, 260, 4099, 1, 8, 4, 0.5),
    (3, 64, 13, 3, 4, 1, 0.0),
    (7, 132, 2051, 1, 12, 0, -0.5),
    (16, 4096, 14336, 0, 0, 0, 0.0),     # K split 32 ways
    (9, 1024, 65536, 4, 4, 2, 0.25),     # split, ragged everything else
    (1, 8192, 8192, 0, 0, 0, 0.0),       # the bench shape
    (4, 2048, 8200, 4, 8, 0, 0.0),       # split, the last slice ending in a partial chunk
    (16, 260, 33, 3, 4, 4, 0.5),         # two full chunks and a 1-row partial one
    (5, 516, 20, 0, 0, 0, -0.5),         # one full chunk and a partial one; 5 column blocks
    (8, 252, 4096, 0, 4, 0, 0.0),        # the second 128-column block partial
    # 17-64 rows: four waves along K, one 64-column group, 2-4 activation tiles
    (17, 1000, 1028, 0, 0, 0, 0.0),
    (20, 68, 13, 3, 4, 2, -0.5),         # one partial chunk only; the second column group partial
    (24, 300, 4100, 4, 4, 1, 0.5),       # K split
    (32, 4096, 4096, 0, 0, 0, 0.0),
    (33, 260, 2051, 1, 8, 0, -0.5),      # the third activation tile one row
    (48, 8192, 1000, 0, 4, 0, 0.0),
    (64, 4096, 4100, 4, 0, 3, 0.25),
    (64, 132, 64, 0, 0, 0, 0.0),         # four chunks, unsplit
]


def _padded(rows, cols, ld, seed, scale):
    """rows x cols fp32 matrix in a buffer of (rows - 1) ld + cols elements,
    NaN in the padding between rows."""
    r = np.random.default_rng(seed)
    buf = np.full((rows - 1) * ld + cols, np.nan, np.float32)
    vals = (r.standard_normal(rows * cols) * scale).astype(np.float32)
    for i in range(rows):
        buf[i * ld: i * ld + cols] = vals[i * cols:(i + 1) * cols]
    return buf


def _run(case, op_b, ex=None):
    import torch
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, f32_bound
    M, N, K, pad_a, pad_b, pad_c, beta = case
    lda, ldc = K + pad_a, N + pad_c
    wrows, wcols = (N, K) if op_b else (K, N)
    ldb = wcols + pad_b
    hX = _padded(M, K, lda, 1 + M + K, 1.0)
    hW = _padded(wrows, wcols, ldb, 2 + N + K, 0.05)
    r = np.random.default_rng(3 + M)
    c = r.standard_normal(M * ldc).astype(np.float32).reshape(M, ldc)
    c[:, N:] = SENT
    hC = c.reshape(-1).copy()
    want = hC.copy()
    alpha = 1.5
    if ex is None:
        oracle.ref_gemm_f32_rm(0, op_b, M, N, K, hX, lda, hW, ldb, alpha, beta, want, ldc)
    else:
        cin = r.standard_normal(M * ldc).astype(np.float32)
        bias = (r.standard_normal(N) * 0.5).astype(np.float32)
        oracle.ref_gemm_epi_rm("f32", "f32", 0, op_b, M, N, K, hX, lda, hW, ldb, alpha, beta,
                               cin if ex["sep"] else want.copy(), ldc, want, ldc, bias)
    dX, dW, dC = to_dev(hX), to_dev(hW), to_dev(hC)
    st = torch.cuda.current_stream().cuda_stream
    pl = vk.plan(vk.DT_F32, vk.DT_F32, 0, op_b, M, N, K, lda, ldb, ldc)
    assert pl.path == vk.PATH_SKINNY
    if ex is None:
        vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, op_b, M, N, K, alpha, dX.data_ptr(), lda, dW.data_ptr(), ldb,
                      beta, dC.data_ptr(), ldc, stream=st)
    else:
        dCin = to_dev(cin) if ex["sep"] else None
        dBias = to_dev(bias)
        vk.gemm_ex_async(vk.DT_F32, vk.DT_F32, vk.OP_N, op_b, M, N, K, alpha, dX.data_ptr(), lda, dW.data_ptr(),
                         ldb, beta, dC.data_ptr(), ldc, c_in=dCin.data_ptr() if dCin is not None else None,
                         ldc_in=ldc if dCin is not None else 0, bias=dBias.data_ptr(), bias_type=vk.DT_F32,
                         stream=st)
    assert vk.last_path() == vk.PATH_SKINNY
    assert vk.last_kernel() == vk.KERNEL_SKINNY
    got = to_host(dC).reshape(M, ldc)
    w = want.reshape(M, ldc)
    assert np.array_equal(got[:, N:], w[:, N:]), "C padding written"
    assert np.all(np.isfinite(got[:, :N]))
    err = normwise(got[:, :N], w[:, :N])
    assert err <= f32_bound(K), err
    return pl.split


@pytest.mark.parametrize("case", CASES_T, ids=lambda c: "M{}_N{}_K{}_pa{}_pb{}_pc{}_b{}".format(*c))
def test_skinny_f32_nk(case):
    """W stored N x K (op_b = T)"""
    print(f"[case] fp32 skinny N x K {case}", flush=True)
    _run(case, 1)


@pytest.mark.parametrize("case", CASES_N, ids=lambda c: "M{}_N{}_K{}_pa{}_pb{}_pc{}_b{}".format(*c))
def test_skinny_f32_kn(case):
    """W stored K x N (op_b = N)"""
    print(f"[case] fp32 skinny K x N {case}", flush=True)
    _run(case, 0)


@pytest.mark.parametrize("op_b", [0, 1])
@pytest.mark.parametrize("M,N,K", [(1, 1000, 1028), (5, 4096, 4100), (16, 256, 8192), (3, 8192, 1000)])
@pytest.mark.parametrize("beta,sep", [(0.0, False), (0.5, False), (-0.75, True)])
def test_skinny_f32_epilogue(op_b, M, N, K, beta, sep):
    """bias and C_in: applied by the kernel, or once by the reduce after a K split"""
    print(f"[case] fp32 skinny epilogue op_b={op_b} M={M} N={N} K={K} beta={beta} sep={sep}", flush=True)
    _run((M, N, K, 4, 4, 4, beta), op_b, ex={"sep": sep})


@pytest.mark.parametrize("op_b", [0, 1])
@pytest.mark.parametrize("M,N,K", [(17, 1000, 4100), (40, 1000, 252), (64, 520, 4100)])
@pytest.mark.parametrize("beta,sep", [(0.0, False), (0.5, False), (-0.75, True)])
def test_decode_f32_epilogue(op_b, M, N, K, beta, sep):
    """17-64 rows: bias and C_in applied by the kernel (K = 252, unsplit) or
    once by the reduce after its K split"""
    print(f"[case] fp32 decode epilogue op_b={op_b} M={M} N={N} K={K} beta={beta} sep={sep}", flush=True)
    _run((M, N, K, 4, 4, 4, beta), op_b, ex={"sep": sep})


@pytest.mark.parametrize("op_b", [0, 1])
@pytest.mark.parametrize("M", [1, 7, 16])
def test_skinny_f32_device_scalars(op_b, M):
    """alpha / beta in device memory (hipBLAS pointer mode device)"""
    import torch
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, f32_bound
    print(f"[case] fp32 skinny device scalars op_b={op_b} M={M}", flush=True)
    N, K = 1024, 4096
    hX = _padded(M, K, K, 11, 1.0)
    hW = _padded(N, K, K, 12, 0.05) if op_b else _padded(K, N, N, 12, 0.05)
    ldb = K if op_b else N
    hC = np.random.default_rng(13).standard_normal(M * N).astype(np.float32)
    want = hC.copy()
    oracle.ref_gemm_f32_rm(0, op_b, M, N, K, hX, K, hW, ldb, 0.75, 0.5, want, N)
    dX, dW, dC = to_dev(hX), to_dev(hW), to_dev(hC)
    sc = torch.tensor([0.75, 0.5], dtype=torch.float32, device="cuda:0")
    vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, op_b, M, N, K, 0.0, dX.data_ptr(), K, dW.data_ptr(), ldb, 0.0,
                  dC.data_ptr(), N, scalar_mode=vk.SCALAR_DEV_F32, alpha_dev=sc.data_ptr(),
                  beta_dev=sc.data_ptr() + 4, stream=torch.cuda.current_stream().cuda_stream)
    assert vk.last_path() == vk.PATH_SKINNY
    assert normwise(to_host(dC), want) <= f32_bound(K)


def test_skinny_f32_deterministic():
    """fixed summation order in both kernels and the split reduce: repeated
    runs are bitwise equal"""
    import torch
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    print("[case] fp32 skinny determinism", flush=True)
    for op_b, M, N, K in ((1, 1, 4096, 8192), (1, 16, 8192, 1024), (0, 1, 8192, 8192), (0, 16, 4096, 14336),
                          (0, 3, 1000, 100), (1, 40, 4096, 4096), (1, 64, 1000, 4100), (0, 40, 4096, 4096),
                          (0, 64, 1000, 4100)):
        ldb = K if op_b else N
        dX = to_dev(_padded(M, K, K, 21, 1.0))
        dW = to_dev(_padded(N, K, K, 22, 0.05) if op_b else _padded(K, N, N, 22, 0.05))
        outs = []
        for _ in range(3):
            dC = torch.empty(M * N, dtype=torch.float32, device="cuda:0")
            vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, op_b, M, N, K, 1.0, dX.data_ptr(), K, dW.data_ptr(), ldb,
                          0.0, dC.data_ptr(), N, stream=torch.cuda.current_stream().cuda_stream)
            assert vk.last_path() == vk.PATH_SKINNY
            outs.append(to_host(dC))
        assert all(np.array_equal(outs[0], o) for o in outs[1:])
