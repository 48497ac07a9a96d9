"""The HIP path against the committed golden fixtures (tests/golden/).

fp32 cases go through hipblasSgemm (column-major, the hipBLAS view of
test/test_gemm.c); fp16 cases through the engine entry point vkblas_gemm_f16
(src/vkblas.h:68-77) and, for fp32 output, vkblas_gemm_async (16F x 16F -> 32F,
the GemmEx combination).  Bars: fp32 normwise <= 1e-5 * sqrt(K); fp16
normwise <= 2e-3; closed-form cases (alpha = 0, K = 1, identity, small
integers) are exact, so they must match bit for bit.
"""
import numpy as np
import pytest

from test_golden import CASES

pytestmark = pytest.mark.gpu

EXACT = {"closed_alpha0", "closed_outer_k1", "closed_identity", "closed_integers"}


@pytest.fixture(scope="module")
def handle():
    from gpu_helpers import Handle
    h = Handle()
    yield h
    h.close()


@pytest.mark.parametrize("case", [c for c in CASES if c[0]["kind"] == "f32cm"], ids=lambda c: c[0]["name"])
def test_sgemm_golden(handle, case):
    from gpu_helpers import to_dev, to_host, fbox, normwise, f32_bound
    from vkblas_amd import hipblas_abi as hb
    meta, a = case
    print(f"[case] golden sgemm {meta['name']}", flush=True)
    dA, dB, dC = to_dev(a["A"]), to_dev(a["B"]), to_dev(a["C"])
    ops = (hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_T)
    st = handle.abi.hipblasSgemm(handle.h, ops[meta["ta"]], ops[meta["tb"]], meta["m"], meta["n"], meta["k"],
                                 fbox(meta["alpha"]), dA.data_ptr(), meta["lda"], dB.data_ptr(), meta["ldb"],
                                 fbox(meta["beta"]), dC.data_ptr(), meta["ldc"])
    assert st == 0
    got = to_host(dC)
    if meta["name"] in EXACT:
        assert np.array_equal(got, a["out"])
    else:
        assert normwise(got, a["out"]) <= f32_bound(meta["k"])
    # entries outside the m rows of each column (padding of ldc) are untouched
    pad = np.ones(got.size, bool)
    for j in range(meta["n"]):
        pad[j * meta["ldc"]: j * meta["ldc"] + meta["m"]] = False
    assert np.array_equal(got[pad], a["C"][pad])


@pytest.mark.parametrize("case", [c for c in CASES if c[0]["kind"] == "f16rm"], ids=lambda c: c[0]["name"])
def test_f16_golden(case):
    import torch
    import oracle
    import vkblas_amd as vk
    from gpu_helpers import to_dev, to_host, normwise, F16_BOUND
    meta, a = case
    print(f"[case] golden f16 {meta['name']}", flush=True)
    M, N, K = meta["M"], meta["N"], meta["K"]
    dA, dB = to_dev(a["A"]), to_dev(a["B"])
    dC = to_dev(a["C"])
    st = vk.gemm_f16(meta["op_a"], meta["op_b"], M, N, K, meta["alpha"], dA.data_ptr(), meta["lda"], dB.data_ptr(),
                     meta["ldb"], meta["beta"], dC.data_ptr(), meta["ldc"])
    assert st == vk.OK
    got = to_host(dC)
    ldc = meta["ldc"]
    idx = (np.arange(M)[:, None] * ldc + np.arange(N)[None, :]).reshape(-1)
    assert normwise(oracle.h2f(got[idx]), oracle.h2f(a["out16"][idx])) <= F16_BOUND
    keep = np.ones(got.size, bool)
    keep[idx] = False
    assert np.array_equal(got[keep], a["C"][keep])
    # fp32 output (GemmEx 16F x 16F -> 32F)
    dCf = to_dev(a["Cf"])
    vk.gemm_async(vk.DT_F16, vk.DT_F32, meta["op_a"], meta["op_b"], M, N, K, meta["alpha"], dA.data_ptr(),
                  meta["lda"], dB.data_ptr(), meta["ldb"], meta["beta"], dCf.data_ptr(), ldc,
                  stream=torch.cuda.current_stream().cuda_stream)
    gotf = to_host(dCf)
    assert normwise(gotf[idx], a["out32"][idx]) <= F16_BOUND
    assert np.array_equal(gotf[keep], a["Cf"][keep])
