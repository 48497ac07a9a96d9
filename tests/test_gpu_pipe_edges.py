"""The pipelined GEMM kernels on shapes whose M and N are not tile multiples.

An edge tile moves back inside the matrix (the last tile row computes rows
M - BM .. M - 1) and stores only the rows / columns the tile before it does
not, so every load stays in bounds and beta != 0 reads each C element once.
Every gemm_pipe_kernel instantiation (256x256; 128x128 in its two- and
four-stage forms) in all four layouts, beta == 0 (C pre-filled with NaN) and
beta != 0, against the CPU oracle:

  n8:  N a multiple of 16 bytes of C: the staged epilogue (16-byte rows);
  n4:  N = 4 mod 8: 16-bit C takes the direct epilogue, and an MN-major
       16-bit B (N not a multiple of 8) the generic kernel.

C sits in a larger buffer: padding columns N..ldc and guard rows after row
M - 1 must come back untouched.  vkblas_last_kernel() checks which kernel
ran.  The row-major engine contract is the reference's src/vkblas.h:21-26;
the reference tests ragged shapes through test/test_gemm.c:231-236
(257x129x64, 100x200x300, 33x65x17).
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

TYPES = [("f32", "f32"), ("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32")]
# tile override, tile edge, M, N (n8 form), K
TILES = {"pipe256": (2, 256, 552, 536, 256), "pipe128x2": (1, 128, 2344, 2328, 128),
         "pipe128x4": (1, 128, 296, 280, 256),
         # M below the 128-row tile: K-major A reads rows past M as row M - 1
         "pipe128short": (1, 128, 100, 280, 256), "pipe128m66": (1, 128, 66, 536, 256)}
GUARD_ROWS = 3


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


def expected_kernel(ab, edge, M, N, op_a, op_b):
    """the launcher's rule: edge tiles need M >= BM (or 128x128 tiles with
    K-major A), N >= BN, N % 4 == 0 and an MN-major operand's ragged dimension
    a multiple of 16 bytes"""
    vec = 4 if ab == "f32" else 8
    ak, bk = op_a == 0, op_b == 1
    m_ok = M >= edge or (edge == 128 and ak)
    if not (m_ok and N >= edge and N % 4 == 0 and (ak or M % vec == 0) and (bk or N % vec == 0)):
        return 2                                  # generic kernel, checked edges
    if edge == 256:
        return 3
    grid = -(-M // 128) * -(-N // 128)
    return 5 if (ab != "f32" and grid <= 256) else 4


def run_edges(ab, ct, tile, op_a, op_b, beta, nform, split_k=1, K=None):
    import vkblas_amd as vk
    from gpu_helpers import normwise, f32_bound, F16_BOUND, BF16_BOUND
    tsel, edge, M, N, K0 = TILES[tile]
    K = K or K0
    if nform == "n4":
        N -= 4
    print(f"[case] pipe edges {ab}>{ct} {tile} op={op_a}{op_b} beta={beta} {nform} M={M} N={N} K={K} "
          f"split={split_k}", flush=True)
    vk.set_override(tsel, False)
    pad = 4 if ab == "f32" else 8
    lda = (M if op_a else K) + pad
    ldb = (K if op_b else N) + pad
    ldc = N + 8
    ca, ba, tda = _conv(ab)
    cc, bc, tdc = _conv(ct)
    a = ca(_uniform(21 + op_a, lda * (K if op_a else M)))
    b = ca(_uniform(23 + op_b, ldb * (N if op_b else K)))
    c0 = _uniform(25, ldc * (M + GUARD_ROWS))
    if beta == 0.0:
        c0.reshape(M + GUARD_ROWS, ldc)[:M, :N] = np.nan
    c = cc(c0)
    full = c.copy()
    rows = None
    if M > 600:
        # the oracle's row sample plus the rows around the edge tile's start
        # (its shifted start M - edge and its own start) and the last rows
        last = (M // edge) * edge
        extra = [M - edge - 1, M - edge, last - 1, last, M - 2, M - 1]
        rows = np.unique(np.concatenate([oracle.sample_rows(M, 12), np.array(extra, np.int32)])).astype(np.int32)
    ref = c[:M * ldc].copy()
    alpha = 0.75
    fn = {("f32", "f32"): oracle.ref_gemm_f32_rm, ("f16", "f16"): oracle.ref_gemm_f16_rm,
          ("f16", "f32"): oracle.ref_gemm_f16f32_rm, ("bf16", "bf16"): oracle.ref_gemm_bf16_rm,
          ("bf16", "f32"): oracle.ref_gemm_bf16f32_rm}[(ab, ct)]
    fn(op_a, op_b, M, N, K, a, lda, b, ldb, alpha, beta, ref, ldc, rows=rows)

    dA, dB, dC = _dev(a, tda), _dev(b, tda), _dev(c, tdc)
    dt = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    vk.gemm_async(dt[ab], dt[ct], op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb, beta,
                  dC.data_ptr(), ldc, split_k=split_k)
    got_all = _host(dC)
    if split_k == 1:
        want_k = expected_kernel(ab, edge, M, N, op_a, op_b)
        assert vk.last_kernel() == want_k, f"kernel {vk.last_kernel()} ran, expected {want_k}"
    g2 = got_all.reshape(M + GUARD_ROWS, ldc)
    f2 = full.reshape(M + GUARD_ROWS, ldc)
    # padding columns of every row and the guard rows after C: untouched
    assert np.array_equal(g2[:, N:].view(np.uint8), f2[:, N:].view(np.uint8))
    assert np.array_equal(g2[M:].view(np.uint8), f2[M:].view(np.uint8))
    sel = np.arange(M) if rows is None else rows
    got = bc(g2[sel, :N]).astype(np.float64)
    want = bc(ref.reshape(M, ldc)[sel, :N]).astype(np.float64)
    assert np.all(np.isfinite(got))
    bound = f32_bound(K) if (ab == "f32") else (BF16_BOUND if ct == "bf16" else F16_BOUND)
    assert normwise(got, want) <= bound
    return vk.last_kernel()


CASES = [(ab, c, t) for (ab, c) in TYPES for t in TILES]


@pytest.mark.parametrize("nform", ["n8", "n4"])
@pytest.mark.parametrize("beta", [0.0, -0.5])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("ab,ct,tile", CASES, ids=[f"{a}>{c}-{t}" for a, c, t in CASES])
def test_pipe_edges(ab, ct, tile, op_a, op_b, beta, nform):
    run_edges(ab, ct, tile, op_a, op_b, beta, nform)


@pytest.mark.parametrize("ab,ct", [("f32", "f32"), ("f16", "f32"), ("bf16", "bf16")])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (1, 1)])
def test_pipe_edges_split_k(ab, ct, op_a, op_b):
    """split-K pass 1 on ragged 128x128 tiles (K = 768 in 3 slices of 256),
    then the reduce with alpha / beta"""
    import vkblas_amd as vk
    kern = run_edges(ab, ct, "pipe128x4", op_a, op_b, -0.5, "n8", split_k=3, K=768)
    assert vk.last_path() == vk.PATH_SPLITK
    # pass 1 on the pipelined kernel (27 workgroups: four stages for 16-bit inputs)
    assert kern == (vk.KERNEL_PIPE128 if ab == "f32" else vk.KERNEL_PIPE128_4), kern


@pytest.mark.parametrize("ab,ct", [("f32", "f32"), ("f16", "f16"), ("bf16", "f32")])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_pipe_edges_strided_batched(ab, ct, op_a, op_b):
    """a strided batch of ragged matrices on the pipelined 128x128 kernel:
    every batch's edge tiles shift inside its own matrix (batch strides with
    a gap between the matrices, which must come back untouched)"""
    import vkblas_amd as vk
    from gpu_helpers import normwise, f32_bound, F16_BOUND, BF16_BOUND
    M, N, K, batch = 296, 264, 256, 3
    print(f"[case] pipe edges batched {ab}>{ct} op={op_a}{op_b} M={M} N={N} K={K} batch={batch}", flush=True)
    vk.set_override(1, False)
    lda = M if op_a else K
    ldb = K if op_b else N
    ldc = N
    sa = lda * (K if op_a else M) + 64
    sb = ldb * (N if op_b else K) + 64
    sc = ldc * M + 64
    ca, ba, tda = _conv(ab)
    cc, bc, tdc = _conv(ct)
    a = ca(_uniform(31 + op_a, sa * batch))
    b = ca(_uniform(33 + op_b, sb * batch))
    c = cc(_uniform(35, sc * batch))
    full = c.copy()
    alpha, beta = 1.25, 0.5
    fn = {("f32", "f32"): oracle.ref_gemm_f32_rm, ("f16", "f16"): oracle.ref_gemm_f16_rm,
          ("bf16", "f32"): oracle.ref_gemm_bf16f32_rm}[(ab, ct)]
    refs = []
    for i in range(batch):
        ref = c[i * sc:i * sc + ldc * M].copy()
        fn(op_a, op_b, M, N, K, a[i * sa:(i + 1) * sa], lda, b[i * sb:(i + 1) * sb], ldb, alpha, beta, ref, ldc)
        refs.append(ref)
    dA, dB, dC = _dev(a, tda), _dev(b, tda), _dev(c, tdc)
    dt = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    vk.gemm_async(dt[ab], dt[ct], op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb, beta,
                  dC.data_ptr(), ldc, batch=batch, stride_a=sa, stride_b=sb, stride_c=sc, split_k=1)
    got = _host(dC)
    # 3 x 9 tiles, fewer workgroups than CUs: four stages for 16-bit inputs, two for fp32
    assert vk.last_kernel() == (vk.KERNEL_PIPE128 if ab == "f32" else vk.KERNEL_PIPE128_4), vk.last_kernel()
    bound = f32_bound(K) if ab == "f32" else (BF16_BOUND if ct == "bf16" else F16_BOUND)
    for i in range(batch):
        g = got[i * sc:(i + 1) * sc]
        f = full[i * sc:(i + 1) * sc]
        assert np.array_equal(g[ldc * M:].view(np.uint8), f[ldc * M:].view(np.uint8))   # gap untouched
        assert normwise(bc(g[:ldc * M]).astype(np.float64), bc(refs[i]).astype(np.float64)) <= bound
