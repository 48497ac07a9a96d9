"""Pointer-array batched GEMM (hipblas*gemmBatched, hipblasGemmBatchedEx and
the engine's vkblas_gemm_batched_async): every batch has its own matrix
pointers, read by the kernels from device arrays.  The reference has no such
entry (it left them to the vendor library), so the oracle is the per-batch
CPU restatement of the plain GEMM.  Matrices sit at scattered offsets in one
buffer, some deliberately misaligned for the vector loads (the kernels check
each batch's alignment), with padded leading dimensions.
Bars: fp32 normwise <= 1e-5 sqrt(K); fp16 and fp32-from-16-bit <= 2e-3; bf16 <= 8e-3.
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

EL = {"f32": 4, "f16": 2, "bf16": 2}


def _place(parts, elem, misalign):
    """Concatenate host arrays into one device buffer at gapped offsets (batch
    b shifted by b % 3 elements when misalign); returns (buffer, pointers, offsets)."""
    offs, pos = [], 0
    for b, a in enumerate(parts):
        pos += (b % 3) if misalign else 0
        offs.append(pos)
        pos += a.size + 17
    host = np.zeros(pos, parts[0].dtype)
    for a, o in zip(parts, offs):
        host[o:o + a.size] = a
    from gpu_helpers import to_dev
    dev = to_dev(host)
    ptrs = torch.tensor([dev.data_ptr() + o * elem for o in offs], dtype=torch.int64, device="cuda:0")
    return dev, ptrs, offs, host


def _conv(dt):
    return oracle.f2bf_rne if dt == "bf16" else oracle.f2h_rne


def _case_inputs(dt, out, nb, M, N, K, lda, ldb, ldc, op_a, op_b, seed):
    r = np.random.default_rng(seed)
    As, Bs, Cs = [], [], []
    for _ in range(nb):
        a = r.uniform(-1, 1, lda * (K if op_a else M)).astype(np.float32)
        b = r.uniform(-1, 1, ldb * (N if op_b else K)).astype(np.float32)
        c = r.uniform(-1, 1, ldc * M).astype(np.float32)
        if dt != "f32":
            a, b = _conv(dt)(a), _conv(dt)(b)
            if out != "f32":
                c = _conv(dt)(c)
        As.append(a); Bs.append(b); Cs.append(c)
    return As, Bs, Cs


def _reference(dt, out, op_a, op_b, M, N, K, a, lda, b, ldb, alpha, beta, c, ldc):
    want = c.copy()
    if dt == "f32":
        oracle.ref_gemm_f32_rm(op_a, op_b, M, N, K, a, lda, b, ldb, alpha, beta, want, ldc)
    elif dt == "f16":
        f = oracle.ref_gemm_f16f32_rm if out == "f32" else oracle.ref_gemm_f16_rm
        f(op_a, op_b, M, N, K, a, lda, b, ldb, alpha, beta, want, ldc)
    else:
        f = oracle.ref_gemm_bf16f32_rm if out == "f32" else oracle.ref_gemm_bf16_rm
        f(op_a, op_b, M, N, K, a, lda, b, ldb, alpha, beta, want, ldc)
    return want


def _check(dt, out, got, want, K):
    from gpu_helpers import normwise, f32_bound, F16_BOUND, BF16_BOUND
    if out == "f32":
        bound = f32_bound(K) if dt == "f32" else F16_BOUND
        assert normwise(got, want) <= bound
    else:
        dec = oracle.bf2f if dt == "bf16" else oracle.h2f
        assert normwise(dec(got), dec(want)) <= (BF16_BOUND if dt == "bf16" else F16_BOUND)


SHAPES = [(96, 80, 64, 5), (257, 130, 75, 3), (512, 512, 256, 4)]
DTS = [("f32", "f32"), ("f16", "f16"), ("f16", "f32"), ("bf16", "bf16"), ("bf16", "f32")]


@pytest.mark.parametrize("dt,out", DTS, ids=[f"{a}>{b}" for a, b in DTS])
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{n}x{k}b{b}" for m, n, k, b in SHAPES])
@pytest.mark.parametrize("misalign", [False, True], ids=["aligned", "misaligned"])
def test_engine_ptr_array(dt, out, op_a, op_b, shape, misalign):
    import vkblas_amd as vk
    from gpu_helpers import to_host
    M, N, K, nb = shape
    print(f"[case] ptr-array {dt}>{out} op={op_a}{op_b} {M}x{N}x{K} batch={nb} misalign={misalign}", flush=True)
    lda = (M if op_a else K) + 8
    ldb = (K if op_b else N) + 8
    ldc = N + 4
    As, Bs, Cs = _case_inputs(dt, out, nb, M, N, K, lda, ldb, ldc, op_a, op_b, 7 + M + op_a + 2 * op_b)
    dA, pA, _, _ = _place(As, EL[dt], misalign)
    dB, pB, _, _ = _place(Bs, EL[dt], misalign)
    dC, pC, oC, hC = _place(Cs, 4 if out == "f32" else 2, misalign)
    dts = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    vk.gemm_batched_async(dts[dt], dts[out], op_a, op_b, M, N, K, 0.75, pA.data_ptr(), lda, pB.data_ptr(), ldb, -0.5,
                          pC.data_ptr(), ldc, nb, stream=torch.cuda.current_stream().cuda_stream)
    got = to_host(dC)
    for b in range(nb):
        want = _reference(dt, out, op_a, op_b, M, N, K, As[b], lda, Bs[b], ldb, 0.75, -0.5, Cs[b], ldc)
        seg = got[oC[b]:oC[b] + ldc * M]
        rows = np.concatenate([np.arange(r * ldc, r * ldc + N) for r in range(M)])
        _check(dt, out, seg[rows], want[rows], K)
        pad = np.ones(ldc * M, bool)
        pad[rows] = False
        assert np.array_equal(seg[pad], Cs[b][pad])          # padding untouched
    # gaps between the matrices untouched
    mask = np.ones(got.size, bool)
    for b in range(nb):
        mask[oC[b]:oC[b] + ldc * M] = False
    assert np.array_equal(got[mask], hC[mask])


@pytest.fixture(scope="module")
def handle():
    from gpu_helpers import Handle
    h = Handle()
    yield h
    h.close()


@pytest.mark.parametrize("api", ["Sgemm", "Hgemm", "Ex_f16_f32", "Ex_bf16", "Ex_f32"])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
def test_hipblas_batched(handle, api, ta, tb):
    """hipBLAS column-major batched calls = engine (op_a = tb, op_b = ta, M = n, N = m, A = B, B = A)."""
    from gpu_helpers import to_host, fbox, hbox
    from vkblas_amd import hipblas_abi as hb
    m, n, k, nb = 130, 70, 96, 4
    dt, out = {"Sgemm": ("f32", "f32"), "Hgemm": ("f16", "f16"), "Ex_f16_f32": ("f16", "f32"),
               "Ex_bf16": ("bf16", "bf16"), "Ex_f32": ("f32", "f32")}[api]
    print(f"[case] hipblas batched {api} {ta}{tb}", flush=True)
    lda, ldb, ldc = (k if ta else m) + 3, (n if tb else k) + 1, m + 2
    # engine view: M = n, N = m, A = hipBLAS B (ld ldb), B = hipBLAS A (ld lda)
    Bs, As, Cs = _case_inputs(dt, out, nb, n, m, k, ldb, lda, ldc, tb, ta, 99 + ta + 2 * tb)
    dA, pA, _, _ = _place(As, EL[dt], True)
    dB, pB, _, _ = _place(Bs, EL[dt], True)
    dC, pC, oC, _ = _place(Cs, 4 if out == "f32" else 2, True)
    handle.set_stream(torch.cuda.current_stream().cuda_stream)
    opA = hb.HIPBLAS_OP_T if ta else hb.HIPBLAS_OP_N
    opB = hb.HIPBLAS_OP_T if tb else hb.HIPBLAS_OP_N
    alpha, beta = 1.25, 0.5
    if api == "Sgemm":
        st = handle.abi.hipblasSgemmBatched(handle.h, opA, opB, m, n, k, fbox(alpha), pA.data_ptr(), lda,
                                            pB.data_ptr(), ldb, fbox(beta), pC.data_ptr(), ldc, nb)
    elif api == "Hgemm":
        st = handle.abi.hipblasHgemmBatched(handle.h, opA, opB, m, n, k, hbox(alpha), pA.data_ptr(), lda,
                                            pB.data_ptr(), ldb, hbox(beta), pC.data_ptr(), ldc, nb)
    else:
        ty = {"f32": hb.HIP_R_32F, "f16": hb.HIP_R_16F, "bf16": hb.HIP_R_16BF}
        st = handle.abi.hipblasGemmBatchedEx(handle.h, opA, opB, m, n, k, fbox(alpha), pA.data_ptr(), ty[dt], lda,
                                             pB.data_ptr(), ty[dt], ldb, fbox(beta), pC.data_ptr(), ty[out], ldc, nb,
                                             hb.HIPBLAS_COMPUTE_32F, hb.HIPBLAS_GEMM_DEFAULT)
    assert st == 0
    got = to_host(dC)
    for b in range(nb):
        want = _reference(dt, out, tb, ta, n, m, k, Bs[b], ldb, As[b], lda, alpha, beta, Cs[b], ldc)
        seg = got[oC[b]:oC[b] + ldc * n]
        cols = np.concatenate([np.arange(j * ldc, j * ldc + m) for j in range(n)])
        _check(dt, out, seg[cols], want[cols], k)


def test_ptr_array_device_scalars():
    import vkblas_amd as vk
    from gpu_helpers import to_host
    M, N, K, nb = 200, 136, 128, 3
    print("[case] ptr-array device scalars", flush=True)
    As, Bs, Cs = _case_inputs("f16", "f16", nb, M, N, K, K, N, N, 0, 0, 5)
    dA, pA, _, _ = _place(As, 2, False)
    dB, pB, _, _ = _place(Bs, 2, False)
    dC, pC, oC, _ = _place(Cs, 2, False)
    sc = torch.tensor([2.0, -1.0], dtype=torch.float32, device="cuda:0")
    vk.gemm_batched_async(vk.DT_F16, vk.DT_F16, 0, 0, M, N, K, 0.0, pA.data_ptr(), K, pB.data_ptr(), N, 0.0,
                          pC.data_ptr(), N, nb, scalar_mode=vk.SCALAR_DEV_F32, alpha_dev=sc.data_ptr(),
                          beta_dev=sc.data_ptr() + 4, stream=torch.cuda.current_stream().cuda_stream)
    got = to_host(dC)
    for b in range(nb):
        want = _reference("f16", "f16", 0, 0, M, N, K, As[b], K, Bs[b], N, 2.0, -1.0, Cs[b], N)
        _check("f16", "f16", got[oC[b]:oC[b] + M * N], want, K)


def test_ptr_array_rejects_null():
    import vkblas_amd as vk
    assert vk.gemm_batched_async(vk.DT_F32, vk.DT_F32, 0, 0, 4, 4, 4, 1.0, None, 4, None, 4, 0.0, None, 4, 1,
                                 check=False) == vk.ERR_PARAM
