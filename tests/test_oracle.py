"""Pins the CPU oracle (oracle/ref_gemm.c) before it is trusted as the checker.

Each oracle function is checked against something it does not share code
with: numpy's float64 matmul, closed forms, exact integer arithmetic, numpy's
IEEE binary16 conversion, glibc rand() called directly -- and each check is
shown to fail on a planted mistake (transposed operand, dropped beta term,
wrong leading dimension, wrong rounding), so it can actually catch one.
"""
import ctypes

import numpy as np
import pytest

import oracle


def rng(seed, n):
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


def _opmat(buf, trans, rows, cols, ld):
    """op(X) (rows x cols) of a column-major buffer with leading dimension ld."""
    if trans:   # X stored cols x rows
        idx = np.arange(rows)[:, None] * ld + np.arange(cols)[None, :]
    else:
        idx = np.arange(rows)[:, None] + np.arange(cols)[None, :] * ld
    return buf[idx].astype(np.float64)


def numpy_gemm_cm(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc):
    """Independent float64 statement of hipBLAS column-major GEMM, with the
    reference's final float step alpha*(float)s + beta*C."""
    s = _opmat(A, ta, m, k, lda) @ _opmat(B, tb, k, n, ldb)
    out = C.copy()
    for j in range(n):
        sl = slice(j * ldc, j * ldc + m)
        out[sl] = np.float32(alpha) * s[:, j].astype(np.float32) + np.float32(beta) * C[sl]
    return out


CM_CASES = [(ta, tb, m, n, k, a, b, pad) for ta in (0, 1) for tb in (0, 1)
            for (m, n, k) in [(3, 5, 7), (33, 65, 17), (1, 64, 64), (64, 1, 64), (20, 30, 1)]
            for (a, b) in [(1.0, 0.0), (0.5, 0.7), (-1.0, 1.0)] for pad in (0, 3)]


@pytest.mark.parametrize("case", CM_CASES)
def test_ref_gemm_cm_matches_numpy(case):
    ta, tb, m, n, k, alpha, beta, pad = case
    lda = (k if ta else m) + pad
    ldb = (n if tb else k) + pad
    ldc = m + pad
    A = rng(1, lda * (m if ta else k))
    B = rng(2, ldb * (k if tb else n))
    C = rng(3, ldc * n)
    got = C.copy()
    oracle.ref_gemm_cm(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, got, ldc)
    want = numpy_gemm_cm(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, C, ldc)
    # both accumulate in double and round once: equal up to one float ulp
    assert np.allclose(got, want, rtol=2e-7, atol=1e-6)
    # and the OpenMP variant is the same arithmetic, bit for bit
    got2 = C.copy()
    oracle.ref_gemm_cm(ta, tb, m, n, k, alpha, A, lda, B, ldb, beta, got2, ldc, threads=4)
    assert np.array_equal(got, got2)


def test_numpy_check_catches_planted_mistakes():
    """The comparison above fails for a transposed operand, a dropped beta
    term or a wrong leading dimension, so it pins those parts."""
    m, n, k = 17, 19, 23
    A, B, C = rng(4, m * k), rng(5, k * n), rng(6, m * n)
    want = numpy_gemm_cm(0, 0, m, n, k, 1.0, A, m, B, k, 0.5, C, m)

    def ok(ta, tb, lda, ldb, beta):
        got = C.copy()
        oracle.ref_gemm_cm(ta, tb, m, n, k, 1.0, A, lda, B, ldb, beta, got, m)
        return np.allclose(got, want, rtol=2e-7, atol=1e-6)

    assert ok(0, 0, m, k, 0.5)
    assert not ok(1, 0, k, k, 0.5)        # transposed A (square-ish ld to stay in bounds)
    assert not ok(0, 0, m, k, 0.0)        # beta term dropped
    assert not ok(0, 0, m - 1, k, 0.5)    # wrong lda


def test_ref_gemm_cm_closed_forms():
    n = 12
    I = np.eye(n, dtype=np.float32).reshape(-1, order="F").copy()
    B = rng(7, n * n)
    C = np.zeros(n * n, np.float32)
    oracle.ref_gemm_cm(0, 0, n, n, n, 1.0, I, n, B, n, 0.0, C, n)
    assert np.array_equal(C, B)                           # I @ B = B
    C = rng(8, n * n)
    C0 = C.copy()
    oracle.ref_gemm_cm(0, 0, n, n, n, 0.0, I, n, B, n, 2.0, C, n)
    assert np.array_equal(C, np.float32(2.0) * C0)        # alpha = 0
    a, b = np.array([3.0], np.float32), np.array([-2.5], np.float32)
    c = np.array([1.0], np.float32)
    oracle.ref_gemm_cm(0, 0, 1, 1, 1, 2.0, a, 1, b, 1, 3.0, c, 1)
    assert c[0] == np.float32(2.0 * 3.0 * -2.5 + 3.0)     # 1x1x1
    # small integers: exact (cf. test/test_cache.c:10-22)
    m, k, nn = 30, 40, 20
    Ai = (np.arange(m * k) % 7).astype(np.float32)
    Bi = ((np.arange(k * nn) * 3) % 5).astype(np.float32)
    Ci = np.zeros(m * nn, np.float32)
    oracle.ref_gemm_cm(0, 0, m, nn, k, 1.0, Ai, m, Bi, k, 0.0, Ci, m)
    exact = Ai.reshape(k, m).T.astype(np.int64) @ Bi.reshape(nn, k).T.astype(np.int64)
    assert np.array_equal(Ci.reshape(nn, m).T, exact.astype(np.float32))


def test_sampling_rule():
    """test_gemm.c:38-43: rows r*m/sample, last row forced to m-1; others untouched."""
    rows = oracle.sample_rows(4096, 12)
    assert list(rows) == [r * 4096 // 12 for r in range(11)] + [4095]
    assert list(oracle.sample_rows(10, 0)) == list(range(10))
    m, n, k = 40, 3, 5
    A, B = rng(9, m * k), rng(10, k * n)
    C = np.full(m * n, 7.0, np.float32)
    oracle.ref_gemm_cm(0, 0, m, n, k, 1.0, A, m, B, k, 0.0, C, m, 12)
    touched = set(oracle.sample_rows(m, 12))
    for i in range(m):
        assert (C[i] != 7.0) == (i in touched)


def test_fill_test_gemm_is_glibc_rand():
    """test_gemm.c:70-73 data, checked against glibc rand() called from Python."""
    libc = ctypes.CDLL("libc.so.6")
    A, B, C = oracle.fill_test_gemm(42, 5, 4, 3)
    libc.srand(42)
    seq = [np.float32(libc.rand() % 200 - 100) / np.float32(10.0) for _ in range(12)]
    assert np.array_equal(np.concatenate([A, B, C]), np.array(seq, np.float32))
    vals = np.concatenate(oracle.fill_test_gemm(7, 1000, 0, 0))
    assert vals.min() >= -10.0 and vals.max() <= 9.9


# ---------------------------------------------------------------- fp16 bits

def test_h2f_exhaustive_vs_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.h2f(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f2h_rne_vs_numpy():
    r = np.random.default_rng(11)
    x = np.concatenate([
        r.standard_normal(200000).astype(np.float32),
        (r.standard_normal(100000) * 1e-5).astype(np.float32),        # subnormal halves
        (r.standard_normal(50000) * 3e4).astype(np.float32),          # near overflow
        # exact ties between neighbouring halves, normal and subnormal
        ((np.arange(0, 4096, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24)),
        ((np.arange(1024, 2048, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10)),
        np.array([65504.0, 65519.99, 65520.0, 1e9, -1e9, 0.0, -0.0, np.inf, -np.inf], np.float32),
        np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32),
    ])
    x = x[~np.isnan(x)]
    got = oracle.f2h_rne(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert oracle.f2h_rne(np.array([np.nan], np.float32))[0] & 0x7c00 == 0x7c00


def test_f2h_check_catches_wrong_rounding():
    """ties-away rounding (the reference's f2h) differs from RNE on ties: the
    numpy comparison above would catch an oracle that rounded that way."""
    ties = ((np.arange(1024, 1100, dtype=np.float32) + 0.5) * np.float32(2.0 ** -10))
    away = np.array([oracle.lib().oracle_f2h_ties_away(float(v)) for v in ties], np.uint16)
    assert not np.array_equal(away, ties.astype(np.float16).view(np.uint16))
    # and away-from-zero is what it claims on those ties
    assert np.array_equal(away, (np.floor(ties * 1024.0) + 1.0).astype(np.float32).__truediv__(1024.0)
                          .astype(np.float16).view(np.uint16))


def test_fill_test_h_is_glibc_rand():
    libc = ctypes.CDLL("libc.so.6")
    libc.rand.restype = ctypes.c_int
    A, _, _ = oracle.fill_test_h(0x5EED, 50, 0, 0)
    libc.srand(0x5EED)
    vals = np.array([np.float32(libc.rand()) / np.float32(2147483647) * np.float32(2.0) - np.float32(1.0)
                     for _ in range(50)], np.float32)
    # the reference rounds these ties away from zero; off ties it equals RNE
    want = vals.astype(np.float16).view(np.uint16)
    assert np.sum(A != want) <= 2
    assert np.all(np.abs(oracle.h2f(A) - vals) <= np.float32(2.0 ** -11))


# ------------------------------------------------------------- fp16 / rm GEMMs

def numpy_rm(op_a, op_b, M, N, K, A, lda, B, ldb):
    if op_a:
        Ae = A[np.arange(K)[None, :] * lda + np.arange(M)[:, None]]
    else:
        Ae = A[np.arange(M)[:, None] * lda + np.arange(K)[None, :]]
    if op_b:
        Be = B[np.arange(N)[None, :] * ldb + np.arange(K)[:, None]]
    else:
        Be = B[np.arange(K)[:, None] * ldb + np.arange(N)[None, :]]
    return Ae.astype(np.float64) @ Be.astype(np.float64)


@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(4, 4, 4), (33, 65, 17), (64, 1, 64), (1, 40, 300)])
def test_ref_gemm_f16_rm_matches_numpy(op_a, op_b, M, N, K):
    lda = (M if op_a else K) + 1
    ldb = (K if op_b else N) + 2
    ldc = N + 1
    A = oracle.f2h_rne(rng(20, lda * (K if op_a else M)))
    B = oracle.f2h_rne(rng(21, ldb * (N if op_b else K)))
    C = oracle.f2h_rne(rng(22, ldc * M))
    got = C.copy()
    oracle.ref_gemm_f16_rm(op_a, op_b, M, N, K, A, lda, B, ldb, 0.75, 0.5, got, ldc)
    s = numpy_rm(op_a, op_b, M, N, K, oracle.h2f(A), lda, oracle.h2f(B), ldb)
    old = oracle.h2f(C).reshape(-1)
    want = C.copy()
    for i in range(M):
        sl = slice(i * ldc, i * ldc + N)
        v = np.float32(0.75) * s[i].astype(np.float32) + np.float32(0.5) * old[sl]
        want[sl] = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    # fp32-output and fp32-input row-major variants agree with the same statement
    got32 = oracle.h2f(C).copy()
    oracle.ref_gemm_f16f32_rm(op_a, op_b, M, N, K, A, lda, B, ldb, 0.75, 0.5, got32, ldc)
    for i in range(M):
        sl = slice(i * ldc, i * ldc + N)
        v = np.float32(0.75) * s[i].astype(np.float32) + np.float32(0.5) * old[sl]
        assert np.array_equal(got32[sl], v)
    g32 = oracle.h2f(C).copy()
    oracle.ref_gemm_f32_rm(op_a, op_b, M, N, K, oracle.h2f(A), lda, oracle.h2f(B), ldb, 0.75, 0.5, g32, ldc)
    assert np.array_equal(g32, got32)


def test_rm_beta_zero_ignores_nan():
    M, N, K = 5, 6, 7
    A, B = rng(30, M * K), rng(31, K * N)
    C = np.full(M * N, np.nan, np.float32)
    oracle.ref_gemm_f32_rm(0, 0, M, N, K, A, K, B, N, 1.0, 0.0, C, N)
    assert np.all(np.isfinite(C))


def test_rm_rows_subset():
    M, N, K = 40, 8, 9
    A, B = rng(32, M * K), rng(33, K * N)
    full = np.zeros(M * N, np.float32)
    part = np.full(M * N, 5.0, np.float32)
    oracle.ref_gemm_f32_rm(0, 0, M, N, K, A, K, B, N, 1.0, 0.0, full, N)
    rows = oracle.sample_rows(M, 12)
    oracle.ref_gemm_f32_rm(0, 0, M, N, K, A, K, B, N, 1.0, 0.0, part, N, rows=rows)
    for r in range(M):
        seg = slice(r * N, (r + 1) * N)
        if r in set(rows):
            assert np.array_equal(part[seg], full[seg])
        else:
            assert np.all(part[seg] == 5.0)


# ---------------------------------------------------------------- bf16 bits

def _torch_bf16_bits(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy() \
        .view(np.uint16)


def test_bf2f_exhaustive_vs_torch():
    import torch
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.bf2f(bits)
    want = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _bf16_probe_values():
    r = np.random.default_rng(12)
    base = r.standard_normal(200000).astype(np.float32)
    # exact ties between neighbouring bf16 values: low half exactly 0x8000,
    # with even and odd kept bits
    tie_bits = (r.integers(0x00800000, 0x7f000000, 20000, dtype=np.uint32) & 0xffff0000) | 0x8000
    ties = np.concatenate([tie_bits, tie_bits | 0x80000000]).view(np.float32)
    return np.concatenate([
        base, base * np.float32(1e-38), base * np.float32(3e38), ties,
        np.array([3.3895314e38, 3.4028235e38, 1e-45, -1e-45, 0.0, -0.0, np.inf, -np.inf], np.float32),
        np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32),
    ])


def test_f2bf_rne_vs_torch():
    """torch's float -> bfloat16 conversion rounds to nearest even; the oracle
    must agree bit for bit on normals, subnormals, ties, overflow and infinities."""
    with np.errstate(over="ignore", invalid="ignore"):
        x = _bf16_probe_values()
    x = x[~np.isnan(x)]
    assert np.array_equal(oracle.f2bf_rne(x), _torch_bf16_bits(x))
    nan = oracle.f2bf_rne(np.array([np.nan, -np.nan], np.float32))
    assert np.all(np.isnan(oracle.bf2f(nan)))


def test_f2bf_check_catches_truncation():
    """Truncating instead of rounding (or rounding ties up) fails the torch
    comparison above on the tie and near-tie probes."""
    with np.errstate(over="ignore", invalid="ignore"):
        x = _bf16_probe_values()
    x = x[np.isfinite(x)]
    want = _torch_bf16_bits(x)
    u = x.view(np.uint32)
    trunc = (u >> 16).astype(np.uint16)
    ties_up = ((u + np.uint32(0x8000)) >> 16).astype(np.uint16)
    assert not np.array_equal(trunc, want)
    assert not np.array_equal(ties_up, want)


@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", [(4, 4, 4), (33, 65, 17), (64, 1, 64), (1, 40, 300)])
def test_ref_gemm_bf16_rm_matches_numpy(op_a, op_b, M, N, K):
    """bf16 GEMM oracle vs numpy float64 on the decoded inputs, rounded by torch."""
    lda = (M if op_a else K) + 1
    ldb = (K if op_b else N) + 2
    ldc = N + 1
    A = oracle.f2bf_rne(rng(40, lda * (K if op_a else M)))
    B = oracle.f2bf_rne(rng(41, ldb * (N if op_b else K)))
    C = oracle.f2bf_rne(rng(42, ldc * M))
    got = C.copy()
    oracle.ref_gemm_bf16_rm(op_a, op_b, M, N, K, A, lda, B, ldb, 0.75, 0.5, got, ldc)
    s = numpy_rm(op_a, op_b, M, N, K, oracle.bf2f(A), lda, oracle.bf2f(B), ldb)
    old = oracle.bf2f(C)
    want = C.copy()
    want32 = old.copy()
    for i in range(M):
        sl = slice(i * ldc, i * ldc + N)
        v = np.float32(0.75) * s[i].astype(np.float32) + np.float32(0.5) * old[sl]
        want[sl] = _torch_bf16_bits(v)
        want32[sl] = v
    assert np.array_equal(got, want)
    got32 = old.copy()
    oracle.ref_gemm_bf16f32_rm(op_a, op_b, M, N, K, A, lda, B, ldb, 0.75, 0.5, got32, ldc)
    assert np.array_equal(got32, want32)


def test_ref_gemm_bf16_closed_forms_and_planted_mistakes():
    """Small integers are exact in bf16 and in the sum: the oracle reproduces
    the integer product, and fails it with a transposed operand, a dropped
    beta term or fp16 decoding of the bf16 inputs."""
    M, N, K = 24, 20, 16
    Ai = ((np.arange(M * K) * 5) % 9 - 4).astype(np.float32)
    Bi = ((np.arange(K * N) * 3) % 7 - 3).astype(np.float32)
    Ci = (np.arange(M * N) % 5).astype(np.float32)
    A, B, C = oracle.f2bf_rne(Ai), oracle.f2bf_rne(Bi), oracle.f2bf_rne(Ci)
    exact = Ai.reshape(M, K).astype(np.int64) @ Bi.reshape(K, N).astype(np.int64) + 2 * Ci.reshape(M, N)
    assert np.abs(exact).max() < 256                    # every result exact in bf16

    def run(op_a, fn=oracle.ref_gemm_bf16_rm, beta=2.0):
        out = C.copy()
        fn(op_a, 0, M, N, K, A, K, B, N, 1.0, beta, out, N)
        return out

    assert np.array_equal(oracle.bf2f(run(0)).reshape(M, N), exact.astype(np.float32))
    assert not np.array_equal(oracle.bf2f(run(1)).reshape(M, N), exact.astype(np.float32))
    assert not np.array_equal(oracle.bf2f(run(0, beta=0.0)).reshape(M, N), exact.astype(np.float32))
    assert not np.array_equal(oracle.bf2f(run(0, fn=oracle.ref_gemm_f16_rm)).reshape(M, N),
                              exact.astype(np.float32))


# ------------------------------------------------------- epilogue (bias, C_in)

def _epi_data(ab, ct, M, N, K, seed):
    rng = np.random.default_rng(seed)
    conv = {"f32": lambda x: x.astype(np.float32), "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}
    a = conv[ab](rng.uniform(-1, 1, M * K).astype(np.float32))
    b = conv[ab](rng.uniform(-1, 1, K * N).astype(np.float32))
    c = conv[ct](rng.uniform(-1, 1, M * N).astype(np.float32))
    return a, b, c


_TYPES = [("f32", "f32"), ("f32", "f16"), ("f32", "bf16"), ("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"),
          ("bf16", "f32")]


@pytest.mark.parametrize("ab,ct", _TYPES)
def test_ref_gemm_epi_reduces_to_in_place_oracles(ab, ct):
    """No bias and C_in == D: the existing restatements, bit for bit."""
    M, N, K = 13, 17, 29
    for op_a in (0, 1):
        for op_b in (0, 1):
            a, b, c = _epi_data(ab, ct, M, N, K, 7 + op_a + 2 * op_b)
            lda, ldb = (M if op_a else K), (K if op_b else N)
            got = c.copy()
            oracle.ref_gemm_epi_rm(ab, ct, op_a, op_b, M, N, K, a, lda, b, ldb, 0.75, -0.5, got, N, got, N)
            want = c.copy()
            if ab == "f32" and ct == "f32":
                oracle.ref_gemm_f32_rm(op_a, op_b, M, N, K, a, lda, b, ldb, 0.75, -0.5, want, N)
            elif ab == "f32":
                # fp32 oracle on the widened C, rounded once
                back, to = (oracle.h2f, oracle.f2h_rne) if ct == "f16" else (oracle.bf2f, oracle.f2bf_rne)
                w32 = back(c).astype(np.float32)
                oracle.ref_gemm_f32_rm(op_a, op_b, M, N, K, a, lda, b, ldb, 0.75, -0.5, w32, N)
                want = to(w32)
            else:
                fn = {("f16", "f16"): oracle.ref_gemm_f16_rm, ("f16", "f32"): oracle.ref_gemm_f16f32_rm,
                      ("bf16", "bf16"): oracle.ref_gemm_bf16_rm, ("bf16", "f32"): oracle.ref_gemm_bf16f32_rm}
                fn[(ab, ct)](op_a, op_b, M, N, K, a, lda, b, ldb, 0.75, -0.5, want, N)
            assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


def test_ref_gemm_epi_closed_forms():
    """A = 0: D = beta * C_in + bias exactly (small integers are exact in
    fp32); C_in separate from D (D's own contents never read); beta == 0
    never reads C_in (NaN there); bias runs along the columns n."""
    M, N, K = 5, 7, 3
    A = np.zeros(M * K, np.float32)
    B = np.arange(K * N, dtype=np.float32)
    cin = np.arange(M * N, dtype=np.float32).reshape(M, N)
    bias = (10 * np.arange(N)).astype(np.float32)
    D = np.full(M * N, 123.0, np.float32)
    oracle.ref_gemm_epi_rm("f32", "f32", 0, 0, M, N, K, A, K, B, N, 1.0, 2.0, cin.reshape(-1), N, D, N, bias)
    assert np.array_equal(D.reshape(M, N), 2.0 * cin + bias[None, :])
    # beta == 0: C_in is never read, the bias alone remains (plus the product)
    A1 = np.ones(M * K, np.float32)
    nan_in = np.full(M * N, np.nan, np.float32)
    D1 = np.zeros(M * N, np.float32)
    oracle.ref_gemm_epi_rm("f32", "f32", 0, 0, M, N, K, A1, K, B, N, 1.0, 0.0, nan_in, N, D1, N, bias)
    want = B.reshape(K, N).sum(axis=0)[None, :] + bias[None, :]
    assert np.array_equal(D1.reshape(M, N), np.broadcast_to(want, (M, N)))
    # padded leading dimensions of C_in and D: the padding is untouched
    ldi, ldd = N + 3, N + 5
    cin_p = np.full(M * ldi, -1.0, np.float32)
    cin_p.reshape(M, ldi)[:, :N] = cin
    D2 = np.full(M * ldd, 77.0, np.float32)
    oracle.ref_gemm_epi_rm("f32", "f32", 0, 0, M, N, K, A, K, B, N, 1.0, 2.0, cin_p, ldi, D2, ldd, bias)
    assert np.array_equal(D2.reshape(M, ldd)[:, :N], 2.0 * cin + bias[None, :])
    assert np.all(D2.reshape(M, ldd)[:, N:] == 77.0)


def test_ref_gemm_epi_planted_mistakes_fail():
    """A bias along the rows, a bias added after the rounding, and C read from
    D instead of C_in are all distinguishable from the oracle."""
    M, N, K = 6, 6, 8
    rng = np.random.default_rng(3)
    a = oracle.f2h_rne(rng.uniform(-1, 1, M * K).astype(np.float32))
    b = oracle.f2h_rne(rng.uniform(-1, 1, K * N).astype(np.float32))
    cin = oracle.f2h_rne(rng.uniform(-1, 1, M * N).astype(np.float32))
    bias = rng.uniform(-1, 1, N).astype(np.float32) * 1e-3 + np.float32(1.0)
    D = np.zeros(M * N, np.uint16)
    oracle.ref_gemm_epi_rm("f16", "f16", 0, 0, M, N, K, a, K, b, N, 1.0, 0.5, cin, N, D, N, bias)
    # float64 model of the definition
    A = oracle.h2f(a).astype(np.float64).reshape(M, K)
    Bm = oracle.h2f(b).astype(np.float64).reshape(K, N)
    s = (A @ Bm).astype(np.float32)
    exact = s + np.float32(0.5) * oracle.h2f(cin).reshape(M, N) + bias[None, :]
    assert np.array_equal(D.reshape(M, N), oracle.f2h_rne(exact.astype(np.float32).reshape(-1)).reshape(M, N))
    rows_bias = s + np.float32(0.5) * oracle.h2f(cin).reshape(M, N) + bias[:, None]
    assert not np.array_equal(D, oracle.f2h_rne(rows_bias.astype(np.float32).reshape(-1)))
    no_bias16 = oracle.f2h_rne((s + np.float32(0.5) * oracle.h2f(cin).reshape(M, N)).astype(np.float32).reshape(-1))
    late = oracle.f2h_rne((oracle.h2f(no_bias16).reshape(M, N) + bias[None, :]).astype(np.float32).reshape(-1))
    assert not np.array_equal(D, late)
    from_d = np.zeros(M * N, np.uint16)
    oracle.ref_gemm_epi_rm("f16", "f16", 0, 0, M, N, K, a, K, b, N, 1.0, 0.5, from_d, N, from_d, N, bias)
    assert not np.array_equal(D, from_d)


@pytest.mark.parametrize("ab,ct", [("f32", "f32"), ("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"),
                                   ("bf16", "f32"), ("f32", "f16")])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_tiled_oracle_equals_plain_loops(ab, ct, op_a, op_b):
    """ref_gemm_tiled_rm (whole-output checks of large shapes) is the plain
    oracle bit for bit: padded leading dimensions, ragged tiles (M, N not
    multiples of its 64 x 256 tiles), alpha and beta, every layout."""
    rng = np.random.default_rng(7 + op_a + 2 * op_b)
    M, N, K = 67, 300, 129
    lda, ldb, ldc = (M if op_a else K) + 3, (K if op_b else N) + 5, N + 2
    cv = {"f32": lambda x: x, "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}
    A = cv[ab](rng.uniform(-1, 1, lda * (K if op_a else M)).astype(np.float32))
    B = cv[ab](rng.uniform(-1, 1, ldb * (N if op_b else K)).astype(np.float32))
    C1 = cv[ct](rng.uniform(-1, 1, ldc * M).astype(np.float32))
    C2 = C1.copy()
    oracle.ref_gemm_epi_rm(ab, ct, op_a, op_b, M, N, K, A, lda, B, ldb, 0.75, -0.5, C1, ldc, C1, ldc)
    oracle.ref_gemm_tiled_rm(ab, ct, op_a, op_b, M, N, K, A, lda, B, ldb, 0.75, -0.5, C2, ldc)
    assert np.array_equal(C1.view(np.uint8), C2.view(np.uint8))
    # and a planted mistake is seen: one k dropped from every sum
    C3 = cv[ct](np.zeros(ldc * M, np.float32))
    oracle.ref_gemm_tiled_rm(ab, ct, op_a, op_b, M, N, K - 1, A, lda, B, ldb, 0.75, 0.0, C3, ldc)
    C4 = cv[ct](np.zeros(ldc * M, np.float32))
    oracle.ref_gemm_tiled_rm(ab, ct, op_a, op_b, M, N, K, A, lda, B, ldb, 0.75, 0.0, C4, ldc)
    assert not np.array_equal(C3.view(np.uint8), C4.view(np.uint8))
