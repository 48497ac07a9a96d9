"""The epilogue inputs of vkblas_gemm_ex_async on every kernel path.

  C = alpha * op(A) op(B) + beta * C_in + bias[n]     (fp32, one rounding)

C_in is a separate matrix with its own leading dimension (hipBLASLt's and
rocBLAS's C != D), bias one value per column n of the row-major C (per row
of hipBLASLt's column-major D: HIPBLASLT_EPILOGUE_BIAS), fp32 / fp16 / bf16.
Every path: the generic kernel (64 / 128 / 256 tiles, checked edges), the
pipelined kernels (256x256, 128x128 in two and four stages), split-K (bias
and C_in applied once, in the reduce), the decode kernels (GEMV, staged
skinny, staged decode with and without a K split) and strided batches (the
bias shared by every batch).  The oracle is oracle.ref_gemm_epi_rm (pinned in
tests/test_oracle.py).  No reference counterpart: the reference's engine had
no epilogue inputs; PyTorch's addmm with a 1-D bias (reference
test/test_torch.py:65-73) is the caller this serves.
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
CONV = {"f32": lambda x: x.astype(np.float32), "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}
BACK = {"f32": lambda x: x.astype(np.float32), "f16": oracle.h2f, "bf16": oracle.bf2f}


def _u(seed, n, scale=1.0):
    return (np.random.default_rng(seed).uniform(-1.0, 1.0, n) * scale).astype(np.float32)


def _dev(x: np.ndarray, t: str) -> torch.Tensor:
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16)).view(TORCH_DT[t]).to("cuda:0")
    return torch.from_numpy(x).to("cuda:0")


def _host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()


@pytest.fixture(autouse=True)
def reset_override():
    import vkblas_amd as vk
    yield
    vk.set_override(-1, False)


def _bound(ab, ct, K):
    from gpu_helpers import f32_bound, F16_BOUND, BF16_BOUND
    if ct == "bf16":
        return BF16_BOUND
    if ct == "f16" or ab != "f32":
        return F16_BOUND
    return f32_bound(K)


def run_case(ab, ct, op_a, op_b, M, N, K, alpha, beta, bias_t, sep_cin, tile=-1, generic=False, split_k=0,
             batch=1, expect_path=None, expect_kernel=None, scale_b=1.0):
    import vkblas_amd as vk
    from gpu_helpers import normwise
    print(f"[case] epi {ab}>{ct} op={op_a}{op_b} {M}x{N}x{K} b={beta} bias={bias_t} sep={sep_cin} tile={tile} "
          f"gen={generic} split={split_k} batch={batch}", flush=True)
    vk.set_override(tile, generic)
    lda = (M if op_a else K) + (8 if sep_cin else 0)
    ldb = (K if op_b else N)
    sa, sb = lda * (K if op_a else M), ldb * (N if op_b else K)
    ldc = N + 4
    ldci = N + 8 if sep_cin else ldc
    sc, sci = ldc * M, ldci * M
    a = CONV[ab](_u(M + 3 * N + K, sa * batch))
    b = CONV[ab](_u(2 * M + N + 5 * K, sb * batch, scale_b))
    cin = CONV[ct](_u(7, sci * batch))
    d0 = CONV[ct](_u(9, sc * batch))
    if not sep_cin:
        d0 = cin.copy()
    bias = None if bias_t is None else CONV[bias_t](_u(11, N))
    want = d0.copy()
    rows = oracle.sample_rows(M, 12) if M > 256 else None
    for bi in range(batch):
        ci = (cin if sep_cin else want)[bi * sci: (bi + 1) * sci].copy()
        dv = want[bi * sc: (bi + 1) * sc].copy()
        oracle.ref_gemm_epi_rm(ab, ct, op_a, op_b, M, N, K, np.ascontiguousarray(a[bi * sa: (bi + 1) * sa]), lda,
                               np.ascontiguousarray(b[bi * sb: (bi + 1) * sb]), ldb, alpha, beta, ci, ldci, dv, ldc,
                               None if bias is None else BACK[bias_t](bias), rows=rows)
        want[bi * sc: (bi + 1) * sc] = dv
    dA, dB, dD = _dev(a, ab), _dev(b, ab), _dev(d0, ct)
    dCin = _dev(cin, ct) if sep_cin else None
    dBias = _dev(bias, bias_t) if bias is not None else None
    dt = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    vk.gemm_ex_async(dt[ab], dt[ct], op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb, beta,
                     dD.data_ptr(), ldc, batch, sa, sb, sc, split_k=split_k,
                     c_in=dCin.data_ptr() if sep_cin else None, ldc_in=ldci if sep_cin else 0,
                     stride_c_in=sci if sep_cin else 0,
                     bias=dBias.data_ptr() if dBias is not None else None,
                     bias_type=dt[bias_t] if bias_t else vk.DT_F32)
    got = _host(dD)
    if expect_path is not None:
        assert vk.last_path() == expect_path
    if expect_kernel is not None:
        assert vk.last_kernel() == expect_kernel, vk.last_kernel()
    if sep_cin:
        assert np.array_equal(_host(dCin).view(np.uint8), cin.view(np.uint8)), "C_in was written"
    sel = np.arange(M) if rows is None else rows
    for bi in range(batch):
        g = BACK[ct](got[bi * sc:(bi + 1) * sc]).reshape(M, ldc)
        w = BACK[ct](want[bi * sc:(bi + 1) * sc]).reshape(M, ldc)
        # the padding columns of D are untouched
        assert np.array_equal(g[:, N:], BACK[ct](d0[bi * sc:(bi + 1) * sc]).reshape(M, ldc)[:, N:])
        assert np.all(np.isfinite(g[sel, :N]))
        assert normwise(g[sel, :N], w[sel, :N]) <= _bound(ab, ct, K), f"batch {bi}"


TYPES = [("f32", "f32"), ("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32"), ("f32", "f16")]
GEN = [(0, True, 2), (1, True, 2), (2, True, 2)]          # tile, generic, expected kernel (checked edges)


@pytest.mark.parametrize("ab,ct", TYPES)
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("beta,sep", [(0.0, False), (-0.5, False), (0.75, True)])
@pytest.mark.parametrize("bias_t", ["f32", "f16", "bf16", None])
def test_generic_edges(ab, ct, op_a, op_b, beta, sep, bias_t):
    """the generic kernel on a ragged shape (checked edges), 128x128 tiles"""
    run_case(ab, ct, op_a, op_b, 200, 136, 72, 0.75, beta, bias_t, sep, tile=1, generic=True, expect_kernel=2)


PIPE = {"pipe256": (2, 3, 512, 256), "pipe128x4": (1, 5, 256, 256), "pipe128x2": (1, 4, 2304, 128)}


@pytest.mark.parametrize("ab,ct", TYPES)
@pytest.mark.parametrize("pipe", list(PIPE))
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (1, 1), (0, 1)])
@pytest.mark.parametrize("beta,sep", [(0.0, False), (0.5, True)])
def test_pipelined(ab, ct, pipe, op_a, op_b, beta, sep):
    tile, kern, M, K = PIPE[pipe]
    if ab == "f32" and kern == 5:
        kern = 4                                 # fp32 128x128 tiles always run two stages
    run_case(ab, ct, op_a, op_b, M, M, K, 1.25, beta, "f16" if ct == "f16" else "f32", sep, tile=tile,
             expect_kernel=kern)


@pytest.mark.parametrize("ab,ct", [("f32", "f32"), ("f16", "f16"), ("bf16", "f32")])
@pytest.mark.parametrize("split", [0, 7])
@pytest.mark.parametrize("beta,sep", [(0.0, False), (0.5, True)])
def test_split_k(ab, ct, split, beta, sep):
    """bias and C_in applied once, by the reduce (pass 1 writes raw sums)"""
    import vkblas_amd as vk
    run_case(ab, ct, 0, 0, 256, 256, 8192, 1.0, beta, ct, sep, split_k=split, expect_path=vk.PATH_SPLITK)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("tokens", [1, 2, 4, 16, 24, 40, 64])
@pytest.mark.parametrize("beta,sep", [(0.0, False), (0.5, True)])
def test_decode(dt, tokens, beta, sep):
    """decode shapes (engine op_a = N, op_b = T): GEMV, staged skinny, staged
    decode (24 tokens at K = 4096 splits K); 40 and 64 tokens: the short-M
    pipelined 128x128 tiles with a K split and the reduce's epilogue"""
    import vkblas_amd as vk
    run_case(dt, dt, 0, 1, tokens, 4096, 4096, 1.0, beta, dt, sep,
             expect_path=vk.PATH_SKINNY if tokens <= 32 else vk.PATH_SPLITK, scale_b=0.05)


@pytest.mark.parametrize("ab,ct", [("f32", "f32"), ("f16", "f16"), ("bf16", "bf16")])
def test_strided_batched_shares_bias(ab, ct):
    run_case(ab, ct, 0, 1, 96, 160, 64, 1.0, 0.5, ct, True, batch=3)


def test_rejects_bad_epilogue_arguments():
    import vkblas_amd as vk
    d = torch.zeros(64, device="cuda:0")
    p = d.data_ptr()
    assert vk.gemm_ex_async(vk.DT_F32, vk.DT_F32, 0, 0, 4, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4, bias=p, bias_type=7,
                            check=False) == vk.ERR_PARAM
    assert vk.gemm_ex_async(vk.DT_F32, vk.DT_F32, 0, 0, 4, 4, 4, 1.0, p, 4, p, 4, 0.0, p, 4, c_in=p, ldc_in=0,
                            check=False) == vk.ERR_PARAM
