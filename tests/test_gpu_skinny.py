"""Edge cases of the decode kernels (engine op_a = N, op_b = T, M <= 64: the
GEMV kernel for M <= 2, the MFMA skinny kernel above, with up to four
16-row activation tiles from M = 17; op_b = N, M <= 16: the K x N kernel;
fp16 and bf16), the path the
reference reaches for matvec / skinny shapes (src/vkblas.c:2100-2392,
2501-2808).  Ragged K (not a multiple of the kernels' K steps), padded
leading dimensions whose padding holds NaN (it must never reach C), beta != 0,
fp32 output and device-memory scalars; the oracle is the fp16 / bf16 CPU
restatement.  Bars: fp16 and fp32 results normwise <= 2e-3, bf16 results
<= 8e-3 (one bf16 ulp).
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

NAN16 = np.uint16(0x7E00)     # quiet NaN, fp16 encoding
NAN_BF16 = np.uint16(0x7FC0)  # quiet NaN, bf16 encoding

CASES = []
for M in (1, 2, 3, 4, 5, 8, 16):
    for (N, K) in ((1, 8), (7, 504), (100, 520), (1000, 1032), (300, 4104), (64, 8192)):
        CASES.append((M, N, K, 0, 0, 0.0, "f16"))
for M in (1, 2, 3, 8, 16):
    for (N, K) in ((7, 504), (1000, 1032), (300, 4104)):
        CASES.append((M, N, K, 0, 0, 0.0, "bf16"))
for M in (17, 31, 32, 47, 64):
    for (N, K) in ((7, 504), (1000, 1032), (300, 4104)):
        CASES.append((M, N, K, 0, 0, 0.0, "f16"))
    CASES.append((M, 520, 2056, 0, 0, 0.0, "bf16"))
CASES += [
    (20, 640, 1000, 8, 24, -0.5, "f16"),
    (33, 333, 4104, 16, 8, 0.75, "f16>f32"),
    (48, 1024, 2048, 0, 0, 0.25, "bf16>f32"),
    (64, 777, 1032, 24, 0, 1.0, "bf16"),
    (1, 1000, 1032, 8, 16, 0.0, "f16"),
    (1, 777, 1000, 16, 8, 0.5, "bf16"),
    (5, 640, 2056, 8, 24, -0.5, "bf16"),
    (2, 1024, 2048, 0, 0, 0.25, "bf16>f32"),
    (12, 512, 520, 8, 0, 1.0, "bf16>f32"),
    (3, 333, 4104, 24, 8, -0.5, "f16"),
    (4, 1024, 2048, 0, 0, 0.25, "f32"),
    (8, 777, 1000, 16, 8, -0.5, "f16"),
    (16, 512, 520, 8, 0, 1.0, "f32"),
    (2, 4096, 4096, 0, 0, 0.0, "f32"),
]
# K not a multiple of 8 (leading dimensions still are): the 8-element group
# that straddles K must not read the NaN padding past it
CASES += [
    (1, 300, 1001, 7, 15, 0.0, "f16"),
    (2, 257, 4099, 5, 13, 0.5, "bf16"),
    (1, 64, 13, 3, 11, 0.0, "f16>f32"),
    (3, 100, 1001, 15, 7, 0.0, "f16"),
    (7, 129, 2051, 13, 5, 0.0, "f16>f32"),
    (16, 64, 13, 3, 11, -0.5, "bf16"),
    (20, 300, 1001, 7, 7, 0.0, "f16"),
    (64, 96, 4099, 13, 5, -0.5, "bf16"),
]
# 9-16 activation rows with at least 8161 weight rows: two weight tiles per
# workgroup (ragged last workgroup, ragged K)
CASES += [
    (12, 8200, 1032, 8, 8, 0.0, "f16"),
    (16, 8192, 520, 0, 0, 0.5, "bf16"),
    (9, 8216, 1001, 7, 15, -0.5, "f16>f32"),
]
# 9-16 activation rows with a longer K on two weight tiles, two waves and
# three stages per wave
CASES += [
    (13, 8300, 6000, 8, 0, 0.5, "f16>f32"),
]
# up to 8 activation rows, at least 512 workgroups and fewer than 64 K steps:
# two waves per workgroup (ragged K tail on the second wave; a single step);
# with 24-40 K steps and 32-row workgroups spreading as evenly as 16-row
# ones, two weight tiles and three stages (the 4104 and 4100 cases)
CASES += [
    (5, 8200, 1032, 8, 8, 0.0, "f16"),
    (8, 8192, 4104, 0, 8, 0.5, "bf16"),
    (3, 8192, 136, 8, 8, -0.5, "f16>f32"),
    (6, 14400, 4100, 4, 12, 0.0, "f16"),
]
# 17-64 activation rows on both decode geometries: R = 2 (128 weight rows per
# workgroup, when its grid fills >= 240 CUs: K split 4, then no split with a
# ragged last workgroup) and R = 1 (64 rows) with a ragged last workgroup;
# the small cases above all take R = 1
CASES += [
    (24, 8192, 2056, 8, 8, 0.0, "f16"),
    (40, 30720, 520, 0, 8, 0.5, "bf16"),
    (17, 30760, 264, 8, 8, 0.0, "f16"),
    (64, 8200, 1032, 8, 0, -0.5, "f16>f32"),
]


def _padded(rows, cols, ld, seed, scale, bf=False):
    """rows x cols fp16 (bf16 if bf) matrix in a buffer of (rows-1)*ld + cols
    elements, NaN in the padding between rows."""
    r = np.random.default_rng(seed)
    buf = np.full((rows - 1) * ld + cols, NAN_BF16 if bf else NAN16, np.uint16)
    conv = oracle.f2bf_rne if bf else oracle.f2h_rne
    vals = conv((r.standard_normal(rows * cols) * scale).astype(np.float32))
    for i in range(rows):
        buf[i * ld: i * ld + cols] = vals[i * cols:(i + 1) * cols]
    return buf


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"M{c[0]}_N{c[1]}_K{c[2]}_pa{c[3]}_pb{c[4]}_b{c[5]}_{c[6]}")
def test_decode_edges(case):
    import torch
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND, BF16_BOUND
    M, N, K, pad_a, pad_b, beta, out = case
    print(f"[case] decode edge {case}", flush=True)
    bf = out.startswith("bf16")
    f32 = out.endswith("f32")
    lda, ldb, ldc = K + pad_a, K + pad_b, N
    hX = _padded(M, K, lda, 1 + M + K, 1.0, bf)
    hW = _padded(N, K, ldb, 2 + N + K, 0.05, bf)
    r = np.random.default_rng(3)
    c = r.standard_normal(M * ldc).astype(np.float32)
    hC = c if f32 else (oracle.f2bf_rne(c) if bf else oracle.f2h_rne(c))
    want = hC.copy()
    if bf:
        ref = oracle.ref_gemm_bf16f32_rm if f32 else oracle.ref_gemm_bf16_rm
    else:
        ref = oracle.ref_gemm_f16f32_rm if f32 else oracle.ref_gemm_f16_rm
    ref(0, 1, M, N, K, hX, lda, hW, ldb, 1.5, beta, want, ldc)
    dX, dW, dC = to_dev(hX), to_dev(hW), to_dev(hC)
    ab = vk.DT_BF16 if bf else vk.DT_F16
    vk.gemm_async(ab, vk.DT_F32 if f32 else ab, vk.OP_N, vk.OP_T, M, N, K, 1.5, dX.data_ptr(), lda,
                  dW.data_ptr(), ldb, beta, dC.data_ptr(), ldc, stream=torch.cuda.current_stream().cuda_stream)
    assert vk.last_path() == vk.PATH_SKINNY
    got = to_host(dC)
    if f32:
        g, w = got, want
    else:
        dec = oracle.bf2f if bf else oracle.h2f
        g, w = dec(got), dec(want)
    assert np.all(np.isfinite(g))
    assert normwise(g, w) <= (BF16_BOUND if bf and not f32 else F16_BOUND)


@pytest.mark.parametrize("M", [1, 4, 12, 40])
def test_decode_device_scalars(M):
    """alpha / beta in device memory (hipBLAS pointer mode device)."""
    import torch
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND
    N, K = 640, 1536
    print(f"[case] decode device scalars M={M}", flush=True)
    hX = _padded(M, K, K, 11, 1.0)
    hW = _padded(N, K, K, 12, 0.05)
    hC = oracle.f2h_rne(np.random.default_rng(13).standard_normal(M * N).astype(np.float32))
    want = hC.copy()
    oracle.ref_gemm_f16_rm(0, 1, M, N, K, hX, K, hW, K, 0.75, 0.5, want, N)
    dX, dW, dC = to_dev(hX), to_dev(hW), to_dev(hC)
    sc = torch.tensor([0.75, 0.5], dtype=torch.float32, device="cuda:0")
    vk.gemm_async(vk.DT_F16, vk.DT_F16, vk.OP_N, vk.OP_T, M, N, K, 0.0, dX.data_ptr(), K, dW.data_ptr(), K, 0.0,
                  dC.data_ptr(), N, scalar_mode=vk.SCALAR_DEV_F32, alpha_dev=sc.data_ptr(),
                  beta_dev=sc.data_ptr() + 4, stream=torch.cuda.current_stream().cuda_stream)
    assert vk.last_path() == vk.PATH_SKINNY
    assert normwise(oracle.h2f(to_host(dC)), oracle.h2f(want)) <= F16_BOUND


def test_decode_deterministic():
    """The decode kernels sum in a fixed order: repeated runs are bitwise equal."""
    import torch
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    print("[case] decode determinism", flush=True)
    # every kernel and geometry: GEMV, staged skinny with one and two weight
    # tiles per workgroup (two tiles for 9-16 and for up to 8 rows), staged
    # decode with 64 and 128 weight rows
    for M, N, K in ((1, 2048, 4096), (3, 2048, 4096), (9, 2048, 4096), (16, 8192, 1024), (8, 8192, 4096),
                    (40, 2048, 4096), (64, 8192, 2048)):
        dX, dW = to_dev(_padded(M, K, K, 21, 1.0)), to_dev(_padded(N, K, K, 22, 0.05))
        outs = []
        for _ in range(3):
            dC = torch.empty(M * N, dtype=torch.float16, device="cuda:0")
            vk.gemm_async(vk.DT_F16, vk.DT_F16, vk.OP_N, vk.OP_T, M, N, K, 1.0, dX.data_ptr(), K, dW.data_ptr(), K,
                          0.0, dC.data_ptr(), N, stream=torch.cuda.current_stream().cuda_stream)
            outs.append(to_host(dC))
        assert all(np.array_equal(outs[0], o) for o in outs[1:])


# Weight stored K x N (engine op_b = N, PyTorch's x @ w): the 16-bit K x N
# kernel for up to 64 activation rows (one to four 16-row tiles), N a
# multiple of 8.  (M, N, K, pad_a,
# pad_b, beta, out): ldb = N + pad_b with NaN in the padding columns; ragged K
# (not a multiple of the 32-row chunk), N not a multiple of the workgroup's
# 256 columns, K split over the grid with fp32 partials and the reduce.
CASES_KN = []
for M in (1, 2, 5, 8, 16):
    for (N, K) in ((8, 32), (264, 1000), (1000, 1032), (4096, 4100)):
        CASES_KN.append((M, N, K, -K % 8, 0, 0.0, "f16"))   # lda a multiple of 8
CASES_KN += [
    (1, 8192, 8192, 0, 0, 0.0, "f16"),       # the bench shape, K split 8 ways
    (16, 8192, 8192, 0, 8, 0.5, "bf16"),
    (3, 2048, 65536, 8, 16, 0.0, "f16>f32"),  # 32 slices
    (9, 520, 33, 7, 8, -0.5, "bf16>f32"),    # one full chunk and one row
    (4, 776, 7, 1, 0, 0.25, "f16"),           # a partial chunk only
    (12, 1032, 2056, 8, 24, 1.0, "bf16"),
    (2, 8, 4104, 0, 8, 0.0, "f32"),
    # 17-64 rows: two to four activation tiles, 128-column workgroups
    (17, 8192, 8192, 0, 0, 0.0, "f16"),
    (24, 1000, 1032, 8, 8, 0.5, "bf16"),
    (33, 264, 4100, 4, 0, 0.0, "f16>f32"),
    (48, 4096, 520, 8, 16, -0.5, "f16"),
    (64, 8192, 2056, 0, 8, 0.25, "bf16>f32"),
    (64, 136, 33, 7, 0, 0.0, "f16"),
    (40, 2048, 65544, 0, 0, 0.0, "bf16"),   # K not in whole 128-element steps: no short-M tiles
]


@pytest.mark.parametrize("case", CASES_KN, ids=lambda c: f"M{c[0]}_N{c[1]}_K{c[2]}_pa{c[3]}_pb{c[4]}_b{c[5]}_{c[6]}")
def test_decode_kn(case):
    import torch
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND, BF16_BOUND
    M, N, K, pad_a, pad_b, beta, out = case
    print(f"[case] decode K x N {case}", flush=True)
    bf = out.startswith("bf16")
    f32 = out.endswith("f32")
    lda, ldb, ldc = K + pad_a, N + pad_b, N
    hX = _padded(M, K, lda, 5 + M + K, 1.0, bf)
    hW = _padded(K, N, ldb, 6 + N + K, 0.05, bf)
    r = np.random.default_rng(7)
    c = r.standard_normal(M * ldc).astype(np.float32)
    hC = c if f32 else (oracle.f2bf_rne(c) if bf else oracle.f2h_rne(c))
    want = hC.copy()
    if bf:
        ref = oracle.ref_gemm_bf16f32_rm if f32 else oracle.ref_gemm_bf16_rm
    else:
        ref = oracle.ref_gemm_f16f32_rm if f32 else oracle.ref_gemm_f16_rm
    ref(0, 0, M, N, K, hX, lda, hW, ldb, 1.5, beta, want, ldc)
    dX, dW, dC = to_dev(hX), to_dev(hW), to_dev(hC)
    ab = vk.DT_BF16 if bf else vk.DT_F16
    pl = vk.plan(ab, vk.DT_F32 if f32 else ab, 0, 0, M, N, K, lda, ldb, ldc)
    assert pl.path == vk.PATH_SKINNY, pl.path
    vk.gemm_async(ab, vk.DT_F32 if f32 else ab, vk.OP_N, vk.OP_N, M, N, K, 1.5, dX.data_ptr(), lda,
                  dW.data_ptr(), ldb, beta, dC.data_ptr(), ldc, stream=torch.cuda.current_stream().cuda_stream)
    assert vk.last_path() == vk.PATH_SKINNY
    got = to_host(dC)
    if f32:
        g, w = got, want
    else:
        dec = oracle.bf2f if bf else oracle.h2f
        g, w = dec(got), dec(want)
    assert np.all(np.isfinite(g))
    assert normwise(g, w) <= (BF16_BOUND if bf and not f32 else F16_BOUND)


@pytest.mark.parametrize("M,N,K", [(1, 1000, 1032), (7, 8192, 8192), (40, 520, 1032), (64, 4096, 2048)])
@pytest.mark.parametrize("sep", [False, True])
def test_decode_kn_epilogue(M, N, K, sep):
    """bias and a separate C input on the K x N kernel: in its own epilogue,
    or once in the reduce after a K split (8192 x 8192)"""
    import torch
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND
    print(f"[case] decode K x N epilogue M={M} N={N} K={K} sep={sep}", flush=True)
    hX = _padded(M, K, K, 31, 1.0)
    hW = _padded(K, N, N, 32, 0.05)
    r = np.random.default_rng(33)
    hC = oracle.f2h_rne(r.standard_normal(M * N).astype(np.float32))
    cin = oracle.f2h_rne(r.standard_normal(M * N).astype(np.float32))
    bias = (r.standard_normal(N) * 0.5).astype(np.float32)
    want = hC.copy()
    oracle.ref_gemm_epi_rm("f16", "f16", 0, 0, M, N, K, hX, K, hW, N, 1.25, -0.5,
                           cin if sep else want.copy(), N, want, N, bias)
    dX, dW, dC, dCin, dB = to_dev(hX), to_dev(hW), to_dev(hC), to_dev(cin), to_dev(bias)
    vk.gemm_ex_async(vk.DT_F16, vk.DT_F16, vk.OP_N, vk.OP_N, M, N, K, 1.25, dX.data_ptr(), K, dW.data_ptr(), N,
                     -0.5, dC.data_ptr(), N, c_in=dCin.data_ptr() if sep else None, ldc_in=N if sep else 0,
                     bias=dB.data_ptr(), bias_type=vk.DT_F32, stream=torch.cuda.current_stream().cuda_stream)
    assert vk.last_path() == vk.PATH_SKINNY
    assert normwise(oracle.h2f(to_host(dC)), oracle.h2f(want)) <= F16_BOUND


def test_decode_kn_deterministic():
    """K x N kernel and its K split: repeated runs are bitwise equal"""
    import torch
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host
    print("[case] decode K x N determinism", flush=True)
    for M, N, K in ((1, 8192, 8192), (16, 4096, 14336), (5, 1000, 1032), (24, 8192, 8192), (64, 1000, 1032)):
        dX, dW = to_dev(_padded(M, K, K, 41, 1.0)), to_dev(_padded(K, N, N, 42, 0.05))
        outs = []
        for _ in range(3):
            dC = torch.empty(M * N, dtype=torch.float16, device="cuda:0")
            vk.gemm_async(vk.DT_F16, vk.DT_F16, vk.OP_N, vk.OP_N, M, N, K, 1.0, dX.data_ptr(), K, dW.data_ptr(), N,
                          0.0, dC.data_ptr(), N, stream=torch.cuda.current_stream().cuda_stream)
            assert vk.last_path() == vk.PATH_SKINNY
            outs.append(to_host(dC))
        assert all(np.array_equal(outs[0], o) for o in outs[1:])
