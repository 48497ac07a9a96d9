"""The reference's fp16 suites through this library's two fp16 boundaries.

* test/test_h.c (engine C API, row-major): vkblas_gemm_f16 on 7 shapes x 4
  (op_a, op_b) with padded ld (lda = K + M%2, ldb = (op_b ? K : N) + N%2,
  ldc = N + K%2), alpha = 1, beta = 0.5, data U[-1,1) after a per-case srand
  (test_h.c:89-152), plus 3 batch shapes x 4 with batch = 4 (test_h.c:160-226).
  Reference bar: max abs error < 0.05 (test_h.c:141, 212).  Here every case
  must succeed (the reference allowed odd ldc to fail, test_h.c:141-143) and
  also meet the north-star bound: normwise relative error <= 2e-3.
* test/test_v9h.c (hipblasGemmEx): 7 boundary cases x {bf16, fp16} with
  values +-[0.5,1) (test_v9h.c:63-128), bar max_rel < 0.02 with
  rel = |got - acc| / (1 + |acc|).  Both types run on this library's kernels
  (the reference routes 16BF GemmEx to its bf16 engine entry,
  src/vkblas_hipblas.c:426-427).
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

H_SHAPES = [(4, 4, 4), (8, 4, 6), (64, 64, 64), (33, 65, 17), (128, 128, 128), (257, 129, 64), (64, 1, 64)]
H_CASES = []
for op_a in (0, 1):
    for op_b in (0, 1):
        for s, (M, N, K) in enumerate(H_SHAPES):
            H_CASES.append((op_a, op_b, M, N, K, 0x5EED + s + 7 * (op_b + 2 * (op_a + 2 * 0))))


def _span(rows, cols, ld):
    return (rows - 1) * ld + cols


@pytest.mark.parametrize("case", H_CASES, ids=[f"fp16 op{c[0]}{c[1]} {c[2]}x{c[3]}x{c[4]}" for c in H_CASES])
def test_gemm_f16_engine(case):
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND
    op_a, op_b, M, N, K, seed = case
    print(f"[case] vkblas_gemm_f16 op_a={op_a} op_b={op_b} {M}x{N}x{K} seed={seed}", flush=True)
    lda = K + (M % 2)
    ldb = (K if op_b else N) + (N % 2)
    ldc = N + (K % 2)
    ba = _span(K if op_a else M, M if op_a else K, lda)
    bb = _span(N if op_b else K, K if op_b else N, ldb)
    bc = _span(M, N, ldc)
    hA, hB, hC = oracle.fill_test_h(seed, ba, bb, bc)
    alpha, beta = 1.0, 0.5
    hR = hC.copy()
    oracle.ref_gemm_f16_rm(op_a, op_b, M, N, K, hA, lda, hB, ldb, alpha, beta, hR, ldc)
    dA, dB, dC = to_dev(hA), to_dev(hB), to_dev(hC)
    rc = vk.gemm_f16(op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb, beta, dC.data_ptr(), ldc)
    assert rc == vk.OK
    hGot = to_host(dC)
    idx = (np.arange(M)[:, None] * ldc + np.arange(N)[None, :]).reshape(-1)
    got = oracle.h2f(hGot[idx])
    want = oracle.h2f(hR[idx])
    maxerr = float(np.max(np.abs(got - want)))
    assert maxerr < 0.05, f"maxerr {maxerr:.3e} (test_h.c bar 0.05)"
    assert normwise(got, want) <= F16_BOUND
    # elements outside the M x N window (row padding) are untouched
    mask = np.ones(bc, bool)
    mask[idx] = False
    assert np.array_equal(hGot[mask], hC[mask])


HB_SHAPES = [(64, 64, 64), (128, 128, 128), (96, 48, 32)]
HB_CASES = []
for op_a in (0, 1):
    for op_b in (0, 1):
        for s, (M, N, K) in enumerate(HB_SHAPES):
            HB_CASES.append((op_a, op_b, M, N, K, 0xBEEF + s + 7 * (op_b + 2 * (op_a + 2 * 0))))


@pytest.mark.parametrize("case", HB_CASES, ids=[f"fp16 batch op{c[0]}{c[1]} {c[2]}x{c[3]}x{c[4]}" for c in HB_CASES])
def test_gemm_f16_engine_batched(case):
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND
    op_a, op_b, M, N, K, seed = case
    NB = 4
    print(f"[case] vkblas_gemm_f16 batch={NB} op_a={op_a} op_b={op_b} {M}x{N}x{K}", flush=True)
    lda, ldb, ldc = K, (K if op_b else N), N
    ba1 = _span(K if op_a else M, M if op_a else K, lda)
    bb1 = _span(N if op_b else K, K if op_b else N, ldb)
    bc1 = _span(M, N, ldc)
    sa, sb, sc = lda * (K if op_a else M), ldb * (N if op_b else K), ldc * M
    ba, bb, bc = ba1 + sa * (NB - 1), bb1 + sb * (NB - 1), bc1 + sc * (NB - 1)
    hA, hB, hC = oracle.fill_test_h(seed, ba, bb, bc)
    alpha, beta = 1.0, 0.5
    hR = hC.copy()
    for b in range(NB):
        Cb = hR[sc * b:]
        oracle.ref_gemm_f16_rm(op_a, op_b, M, N, K, hA[sa * b:], lda, hB[sb * b:], ldb, alpha, beta, Cb, ldc)
    dA, dB, dC = to_dev(hA), to_dev(hB), to_dev(hC)
    rc = vk.gemm_f16(op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb, beta, dC.data_ptr(), ldc,
                     NB, sa, sb, sc)
    assert rc == vk.OK
    hGot = to_host(dC)
    got, want = oracle.h2f(hGot), oracle.h2f(hR)
    assert float(np.max(np.abs(got - want))) < 0.05
    assert normwise(got, want) <= F16_BOUND


V9H_CASES = [(256, 256, 256, 256, 256, 256, 0, 1), (130, 258, 70, 74, 72, 260, 0, 1),
             (256, 256, 256, 256, 256, 256, 1, 0), (130, 258, 70, 130, 258, 260, 1, 0),
             (130, 258, 70, 74, 260, 260, 0, 0), (256, 512, 256, 256, 512, 512, 0, 1),
             (64, 64, 48, 48, 64, 64, 0, 1)]


def _v9h_data(sa, sb, seed):
    """test_v9h.c:81-93: values +-[0.5, 1) as raw 16-bit patterns from rand()."""
    import ctypes
    libc = ctypes.CDLL("libc.so.6")
    libc.srand(seed)
    out = []
    for n in (sa, sb):
        v = np.empty(n, np.uint16)
        for i in range(n):
            x = libc.rand() % 0x0400 + 0x3800
            if libc.rand() & 1:
                x |= 0x8000
            v[i] = x
        out.append(v)
    return out


def _bf16_to_f32(h):
    return (h.astype(np.uint32) << 16).view(np.float32)


@pytest.mark.parametrize("dtype", ["bf16", "f16"])
@pytest.mark.parametrize("ci", range(len(V9H_CASES)))
def test_gemmex_v9h(dtype, ci):
    """test_v9h.c main loop (lines 74-136) through hipblasGemmEx."""
    import torch
    from vkblas_amd import hipblas_abi as hb
    from gpu_helpers import Handle, to_dev, to_host, fbox
    M, N, K, lda, ldb, ldc, ta, tb = V9H_CASES[ci]
    d = 0 if dtype == "bf16" else 1
    print(f"[case] hipblasGemmEx {dtype} {M}x{N}x{K} ta={ta} tb={tb}", flush=True)
    sa = (K if ta else M) * lda
    sb = (N if tb else K) * ldb
    hA, hB = _v9h_data(sa, sb, 777 + d * 100 + ci)
    dA, dB = to_dev(hA), to_dev(hB)
    dC = torch.zeros(M * ldc, dtype=torch.float16, device="cuda:0")
    dt = hb.HIP_R_16BF if d == 0 else hb.HIP_R_16F
    h = Handle()
    try:
        st = h.abi.hipblasGemmEx(h.h, hb.HIPBLAS_OP_T if tb else hb.HIPBLAS_OP_N,
                                 hb.HIPBLAS_OP_T if ta else hb.HIPBLAS_OP_N, N, M, K, fbox(1.0), dB.data_ptr(), dt,
                                 ldb, dA.data_ptr(), dt, lda, fbox(0.0), dC.data_ptr(), dt, ldc,
                                 hb.HIPBLAS_COMPUTE_32F, hb.HIPBLAS_GEMM_DEFAULT)
    finally:
        h.close()
    assert st == 0
    hC = to_host(dC)
    conv = _bf16_to_f32 if d == 0 else oracle.h2f
    fA = conv(hA).astype(np.float64)
    fB = conv(hB).astype(np.float64)
    i = np.arange(M)[:, None]
    kk = np.arange(K)[None, :]
    Aeff = fA[(kk * lda + i) if ta else (i * lda + kk)]            # M x K
    j = np.arange(N)[None, :]
    kk2 = np.arange(K)[:, None]
    Beff = fB[(j * ldb + kk2) if tb else (kk2 * ldb + j)]          # K x N
    acc = Aeff @ Beff
    got = conv(hC.reshape(M, ldc)[:, :N]).astype(np.float64)
    rel = np.abs(got - acc) / (1.0 + np.abs(acc))
    assert float(rel.max()) < 0.02
