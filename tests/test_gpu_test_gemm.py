"""The reference's fp32 correctness suite, test/test_gemm.c, through the
hipBLAS ABI of libvkblas_hipblas.so.

Case list, seeds, data and pass rule follow test/test_gemm.c:224-293 (17 shapes
x 4 transpose variants with tight ld, 3 alpha/beta/padded-ld specials, 5 batch
shapes x 4 variants, 3 batch specials with stride-0 broadcast); data are
(rand()%200-100)/10 after srand(seed) (test_gemm.c:70-73); the oracle is
ref_gemm (test_gemm.c:32-58) with its 12-row sampling when m*n*k > 5e6
(test_gemm.c:87), pass iff maxdiff < 0.1 (test_gemm.c:117).  On top, the
normwise relative error <= 1e-5 * sqrt(K).
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

SHAPES = [(32, 32, 32), (64, 64, 64), (128, 128, 128), (257, 129, 64), (100, 200, 300),
          (256, 256, 4096), (512, 512, 4096), (512, 640, 4096), (512, 768, 4096),
          (4096, 4096, 4096), (4096, 1024, 4096), (1024, 4096, 4096), (512, 512, 512),
          (33, 65, 17), (1, 64, 64), (64, 1, 64), (3, 5, 7)]

CASES = []
for s, (m, n, k) in enumerate(SHAPES):
    for ta in (0, 1):
        for tb in (0, 1):
            lda = k if ta else m
            ldb = n if tb else k
            CASES.append((f"{'NT'[ta]}{'NT'[tb]} {m}x{n}x{k}", ta, tb, m, n, k, lda, ldb, m, 1.0, 0.0,
                          42 + s * 10 + ta * 2 + tb))
CASES += [
    ("alpha=0.5 beta=0.7", 1, 1, 256, 128, 64, 64, 128, 256, 0.5, 0.7, 7),
    ("padded lda=140 ldb=80 ldc=300", 0, 1, 128, 64, 64, 140, 80, 300, 1.0, 0.0, 8),
    ("padded both T", 1, 1, 100, 50, 80, 120, 90, 150, 1.0, 1.0, 9),
]

BSHAPES = [(64, 64, 64, 64, 64, 64, 4096, 4096, 4096, 8),
           (128, 128, 128, 128, 128, 128, 16384, 16384, 16384, 6),
           (256, 256, 256, 256, 256, 256, 65536, 65536, 65536, 4),
           (33, 65, 17, 40, 70, 40, 2800, 1190, 2600, 5),
           (100, 200, 300, 320, 310, 110, 32000, 62000, 22000, 3)]
BCASES = []
for s, (m, n, k, lda, ldb, ldc, sa, sb, sc, nb) in enumerate(BSHAPES):
    for ta in (0, 1):
        for tb in (0, 1):
            BCASES.append((f"{'NT'[ta]}{'NT'[tb]} {m}x{n}x{k}", ta, tb, m, n, k, lda, ldb, ldc, sa, sb, sc, nb,
                           1.0, 0.0, 100 + s * 10 + ta * 2 + tb))
BCASES += [
    ("alpha=0.5 beta=0.7 b=4", 0, 0, 64, 64, 64, 64, 64, 64, 4096, 4096, 4096, 4, 0.5, 0.7, 7),
    ("broadcast strideA=0", 0, 0, 96, 48, 32, 96, 32, 96, 0, 1536, 4608, 6, 1.0, 0.0, 8),
    ("broadcast strideB=0", 1, 1, 48, 96, 32, 32, 96, 48, 1536, 0, 4608, 6, 1.0, 1.0, 9),
]

OPS = None


def _ops():
    from vkblas_amd import hipblas_abi as hb
    return (hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_T)


@pytest.fixture(scope="module")
def handle():
    from gpu_helpers import Handle
    h = Handle()
    yield h
    h.close()


def _check(hRef, hGot, rows, m, n, ldc, k, offsets=(0,)):
    from gpu_helpers import f32_bound
    maxd = 0.0
    refv, gotv = [], []
    for off in offsets:
        for i in rows:
            r = hRef[off + i + np.arange(n) * ldc]
            g = hGot[off + i + np.arange(n) * ldc]
            maxd = max(maxd, float(np.max(np.abs(r.astype(np.float64) - g))))
            refv.append(r)
            gotv.append(g)
    ref = np.concatenate(refv).astype(np.float64)
    got = np.concatenate(gotv).astype(np.float64)
    rel = float(np.max(np.abs(ref - got)) / max(np.max(np.abs(ref)), 1e-30))
    assert maxd < 0.1, f"maxdiff {maxd:.3e} (test_gemm.c bar 0.1)"
    assert rel <= f32_bound(k), f"normwise {rel:.3e} > 1e-5*sqrt(K)={f32_bound(k):.3e}"
    return maxd, rel


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_sgemm_case(handle, case):
    """test_gemm.c run_case (lines 60-126) through hipblasSgemm."""
    from gpu_helpers import to_dev, to_host, fbox
    name, ta, tb, m, n, k, lda, ldb, ldc, alpha, beta, seed = case
    print(f"[case] sgemm {name} seed={seed}", flush=True)
    szA = lda * m if ta else lda * k
    szB = ldb * k if tb else ldb * n
    szC = ldc * n
    hA, hB, hC = oracle.fill_test_gemm(seed, szA, szB, szC)
    sample = 12 if m * n * k > 5000000 else 0
    hRef = hC.copy()
    oracle.ref_gemm_cm(ta, tb, m, n, k, alpha, hA, lda, hB, ldb, beta, hRef, ldc, sample, threads=0)
    dA, dB, dC = to_dev(hA), to_dev(hB), to_dev(hC)
    ops = _ops()
    st = handle.abi.hipblasSgemm(handle.h, ops[ta], ops[tb], m, n, k, fbox(alpha), dA.data_ptr(), lda,
                                 dB.data_ptr(), ldb, fbox(beta), dC.data_ptr(), ldc)
    assert st == 0
    hGot = to_host(dC)
    rows = oracle.sample_rows(m, sample)
    _check(hRef, hGot, rows, m, n, ldc, k)
    # padding rows of C (ldc > m) are never written
    if ldc > m:
        pad = np.ones(szC, bool)
        for j in range(n):
            pad[j * ldc: j * ldc + m] = False
        assert np.array_equal(hGot[pad], hC[pad])


@pytest.mark.parametrize("case", BCASES, ids=[c[0] for c in BCASES])
def test_sgemm_strided_batched_case(handle, case):
    """test_gemm.c run_batch_case (lines 129-205) through hipblasSgemmStridedBatched."""
    from gpu_helpers import to_dev, to_host, fbox
    name, ta, tb, m, n, k, lda, ldb, ldc, sa, sb, sc, nb, alpha, beta, seed = case
    print(f"[case] sgemm_strided_batched {name} batch={nb} seed={seed}", flush=True)
    szA1 = lda * m if ta else lda * k
    szB1 = ldb * k if tb else ldb * n
    szC1 = ldc * n
    szA = (sa * (nb - 1) if sa > 0 else 0) + szA1
    szB = (sb * (nb - 1) if sb > 0 else 0) + szB1
    szC = (sc * (nb - 1) if sc > 0 else 0) + szC1
    hA, hB, hC = oracle.fill_test_gemm(seed, szA, szB, szC)
    hRef = hC.copy()
    sample = 12 if m * n * k > 5000000 else 0
    for b in range(nb):
        Ab = hA[(sa * b if sa > 0 else 0):]
        Bb = hB[(sb * b if sb > 0 else 0):]
        Cb = hRef[(sc * b if sc > 0 else 0):]
        Cb = np.ascontiguousarray(Cb)
        oracle.ref_gemm_cm(ta, tb, m, n, k, alpha, np.ascontiguousarray(Ab), lda, np.ascontiguousarray(Bb), ldb,
                           beta, Cb, ldc, sample, threads=0)
        hRef[(sc * b if sc > 0 else 0):] = Cb
    dA, dB, dC = to_dev(hA), to_dev(hB), to_dev(hC)
    ops = _ops()
    st = handle.abi.hipblasSgemmStridedBatched(handle.h, ops[ta], ops[tb], m, n, k, fbox(alpha), dA.data_ptr(),
                                               lda, sa, dB.data_ptr(), ldb, sb, fbox(beta), dC.data_ptr(), ldc, sc,
                                               nb)
    assert st == 0
    hGot = to_host(dC)
    # test_gemm.c compares the whole C buffer when not sampling (lines 190-195)
    if sample == 0:
        assert float(np.max(np.abs(hRef.astype(np.float64) - hGot))) < 0.1
    rows = oracle.sample_rows(m, sample)
    _check(hRef, hGot, rows, m, n, ldc, k, offsets=[(sc * b if sc > 0 else 0) for b in range(nb)])
