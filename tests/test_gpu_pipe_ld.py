"""The pipelined GEMM kernels with padded leading dimensions and offset C.

Every gemm_pipe_kernel instantiation (256x256 and 128x128, fp32 and 16-bit;
16-bit 128x128 in its two- and four-stage forms) in all four layouts, beta == 0 (C pre-filled
with NaN, never read) and beta != 0, against the CPU oracle, with operands the
way PyTorch hands over views: lda / ldb = dim + 8 (fp32: + 4, still whole
16-byte chunks per row, so the DMA path takes them), and C as

  ld16:  ldc = N + 8 (fp32: N + 4): rows 16-byte aligned, staged epilogue;
  ldc4:  ldc = N + 4 for 16-bit C (rows alternate between 16- and 8-byte
         alignment), direct epilogue;
  off8:  C starts 8 bytes into its buffer, ldc = N + 8: 16-bit C takes the
         direct epilogue, fp32 C (no 16-byte vector stores possible) the
         checked generic kernel.

vkblas_last_kernel() checks which kernel ran.  The padding of C (columns
N..ldc and the bytes in front of C) must come back untouched.  The row-major
engine contract is the reference's src/vkblas.h:21-26; padded leading
dimensions are exercised by its test_gemm.c:283-285.
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

# (ab, c): element types of A/B and of C
TYPES = [("f32", "f32"), ("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32")]
# tile override, expected kernel, M = N, K
TILES = {"pipe256": (2, 3, 512, 256), "pipe128x4": (1, 5, 256, 256), "pipe128x2": (1, 4, 2304, 128)}
CASES = [(ab, c, t) for (ab, c) in TYPES for t in TILES]


def _uniform(seed, n):
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


@pytest.fixture(autouse=True)
def reset_override():
    import vkblas_amd as vk
    yield
    vk.set_override(-1, False)


def _conv(t):
    if t == "f16":
        return oracle.f2h_rne, oracle.h2f, torch.float16
    if t == "bf16":
        return oracle.f2bf_rne, oracle.bf2f, torch.bfloat16
    return (lambda x: x), (lambda x: x), torch.float32


def _dev(bits: np.ndarray, dt) -> torch.Tensor:
    if bits.dtype == np.uint16:
        return torch.from_numpy(bits.view(np.int16)).view(dt).to("cuda:0")
    return torch.from_numpy(bits).to("cuda:0")


def _host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()


@pytest.mark.parametrize("cpad", ["ld16", "ldc4", "off8"])
@pytest.mark.parametrize("beta", [0.0, -0.5])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("ab,ct,tile", CASES, ids=[f"{a}>{c}-{t}" for a, c, t in CASES])
def test_pipe_padded(ab, ct, tile, op_a, op_b, beta, cpad):
    import vkblas_amd as vk
    from gpu_helpers import normwise, f32_bound, F16_BOUND, BF16_BOUND
    if cpad == "ldc4" and ct == "f32":
        pytest.skip("fp32 C with ldc % 4 == 0 is always 16-byte rows (the ld16 case)")
    tsel, kern, M, K = TILES[tile]
    N = M
    pad = 4 if ab == "f32" else 8
    print(f"[case] pipe padded {ab}>{ct} {tile} op={op_a}{op_b} beta={beta} cpad={cpad}", flush=True)
    vk.set_override(tsel, False)
    lda = (M if op_a else K) + pad
    ldb = (K if op_b else N) + pad
    cv = 4 if ct == "f32" else 8                 # elements per 16 bytes of C
    ldc = N + (4 if cpad == "ldc4" else cv)
    off = 0 if cpad != "off8" else (2 if ct == "f32" else 4)   # elements in front of C (8 bytes)
    if ab == "f32" and kern == 5:
        kern = 4                                 # fp32 128x128 tiles always run two stages
    expect = 2 if (cpad == "off8" and ct == "f32") else kern

    ca, ba, tda = _conv(ab)
    cc, bc, tdc = _conv(ct)
    a = ca(_uniform(1 + op_a, lda * (K if op_a else M)))
    b = ca(_uniform(3 + op_b, ldb * (N if op_b else K)))
    c0 = _uniform(5, off + ldc * M)
    if beta == 0.0:
        c0[off:].reshape(M, ldc)[:, :N] = np.nan
    c = cc(c0)
    full = c.copy()
    rows = oracle.sample_rows(M, 12) if M > 512 else None
    ref = c[off:].copy()
    alpha = 0.75
    fn = {("f32", "f32"): oracle.ref_gemm_f32_rm, ("f16", "f16"): oracle.ref_gemm_f16_rm,
          ("f16", "f32"): oracle.ref_gemm_f16f32_rm, ("bf16", "bf16"): oracle.ref_gemm_bf16_rm,
          ("bf16", "f32"): oracle.ref_gemm_bf16f32_rm}[(ab, ct)]
    fn(op_a, op_b, M, N, K, a, lda, b, ldb, alpha, beta, ref, ldc, rows=rows)

    dA, dB, dC = _dev(a, tda), _dev(b, tda), _dev(c, tdc)
    dt = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    cptr = dC.data_ptr() + off * dC.element_size()
    vk.gemm_async(dt[ab], dt[ct], op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb, beta,
                  cptr, ldc, split_k=1)
    got_all = _host(dC)
    assert vk.last_kernel() == expect, f"kernel {vk.last_kernel()} ran, expected {expect}"
    # padding untouched: bytes in front of C and columns N..ldc of every row
    assert np.array_equal(got_all[:off].view(np.uint8), full[:off].view(np.uint8))
    g2 = got_all[off:].reshape(M, ldc)
    f2 = full[off:].reshape(M, ldc)
    assert np.array_equal(g2[:, N:].view(np.uint8), f2[:, N:].view(np.uint8))
    sel = np.arange(M) if rows is None else rows
    got = bc(g2[sel, :N]).astype(np.float64)
    want = bc(ref.reshape(M, ldc)[sel, :N]).astype(np.float64)
    assert np.all(np.isfinite(got))
    bound = f32_bound(K) if (ab == "f32") else (BF16_BOUND if ct == "bf16" else F16_BOUND)
    assert normwise(got, want) <= bound
