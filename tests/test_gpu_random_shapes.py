"""Seeded random sweep over the engine's argument space, every result checked
against the oracle (oracle.ref_gemm_epi_rm, pinned in tests/test_oracle.py).

Each case draws the input / output types (every pair the engine takes), both
transposes, a shape class (decode rows against a weight, tiles with ragged
edges, large outputs, few tiles with a long K, strided batches), aligned or
ragged dimensions, padded leading dimensions whose padding holds NaN, alpha and beta (beta == 0 over a C full of NaN,
which must not reach the result), sometimes a caller's K split, a separate C
input and a bias.  The planner then picks the path (GEMV, staged decode,
K x N decode, generic, pipelined 128 / 256 tiles, split tail, split-K in its
forms); the sweep reaches combinations the hand-written cases name one by
one.  The reference's own tests check fixed shapes (test/test_gemm.c:129-205,
test/test_h.c:60-140); this widens them.  Bars as elsewhere: fp32 results of
fp32 inputs normwise <= 1e-5 sqrt(K), fp16 results and 16-bit inputs with
fp32 results <= 2e-3, bf16 results <= 8e-3; large outputs are compared on 16
sampled rows (oracle.sample_rows, test_gemm.c's practice).
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

NCASES = 400
PAIRS = [("f32", "f32"), ("f32", "f16"), ("f32", "bf16"), ("f16", "f16"), ("f16", "f32"),
         ("bf16", "bf16"), ("bf16", "f32")]
NAN = {"f32": np.float32(np.nan), "f16": np.uint16(0x7E00), "bf16": np.uint16(0x7FC0)}
CONV = {"f32": lambda x: x.astype(np.float32), "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}
BACK = {"f32": lambda x: x.astype(np.float32), "f16": oracle.h2f, "bf16": oracle.bf2f}


def _draw(i):
    """Case i: a dict of the call's arguments, from a generator seeded by i."""
    r = np.random.default_rng(1000 + i)
    ab, ct = PAIRS[r.integers(len(PAIRS))]
    cls = str(r.choice(["decode", "tiles", "large", "longk", "batched"], p=[0.3, 0.3, 0.1, 0.15, 0.15]))
    if cls == "decode":
        M, N, K = int(r.integers(1, 65)), int(r.integers(1, 3000)), int(r.integers(1, 6000))
    elif cls == "tiles":
        M, N, K = int(r.integers(65, 1100)), int(r.integers(65, 1100)), int(r.integers(1, 2500))
    elif cls == "large":
        M, N, K = int(r.integers(2000, 4400)), int(r.integers(2000, 4400)), int(r.integers(64, 1100))
    elif cls == "longk":
        M, N, K = int(r.integers(1, 300)), int(r.integers(1, 300)), int(r.integers(2048, 20000))
    else:
        M, N, K = int(r.integers(1, 400)), int(r.integers(1, 400)), int(r.integers(1, 700))
    # most calls in models are aligned (dimensions and leading dimensions in
    # whole 16-byte groups, K in whole 128-element steps), which is what the
    # pipelined and decode kernels take; the rest are ragged anywhere
    aligned = r.random() < 0.65
    if aligned:
        M = M if M <= 64 else -(-M // 8) * 8
        N = -(-N // 8) * 8
        K = -(-K // 128) * 128 if r.random() < 0.7 else -(-K // 8) * 8

    def pad():
        if aligned:
            return 0 if r.random() < 0.7 else 8 * int(r.integers(1, 5))
        return 0 if r.random() < 0.5 else int(r.integers(1, 18))
    case = dict(i=i, ab=ab, ct=ct, cls=cls, M=M, N=N, K=K, op_a=int(r.integers(2)), op_b=int(r.integers(2)),
                pa=pad(), pb=pad(), pc=pad(), batch=int(r.integers(2, 4)) if cls == "batched" else 1,
                alpha=float(np.round(r.uniform(-2, 2), 3)),
                beta=0.0 if r.random() < 0.5 else float(np.round(r.uniform(-1.5, 1.5), 3)),
                split=int(r.integers(2, 10)) if cls != "batched" and r.random() < 0.2 else 0,
                cin=bool(r.random() < 0.15), bias=bool(r.random() < 0.2))
    return case


CASES = [_draw(i) for i in range(NCASES)]


def _id(c):
    return (f"{c['i']}_{c['cls']}_{c['ab']}-{c['ct']}_{'TN'[c['op_a']]}{'TN'[c['op_b']]}_"
            f"M{c['M']}N{c['N']}K{c['K']}b{c['batch']}s{c['split']}")


def _mats(r, nb, stride, rows, cols, ld, t, scale):
    """nb rows x cols matrices (row-major, pitch ld) at a stride of `stride`
    elements, in type t, NaN in every gap and padding."""
    buf = np.full(nb * stride, NAN[t], np.float32 if t == "f32" else np.uint16)
    for b in range(nb):
        vals = CONV[t]((r.standard_normal(rows * cols) * scale).astype(np.float32)).reshape(rows, cols)
        view = buf[b * stride: b * stride + rows * ld].reshape(rows, ld)
        view[:, :cols] = vals
    return buf


@pytest.mark.parametrize("c", CASES, ids=_id)
def test_random_shape(c):
    import torch
    import vkblas_amd as vk
    from gpu_helpers import normwise, f32_bound, F16_BOUND, BF16_BOUND
    print(f"[case] random {_id(c)} {c}", flush=True)
    DT = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
    ab, ct, M, N, K, op_a, op_b, nb = c["ab"], c["ct"], c["M"], c["N"], c["K"], c["op_a"], c["op_b"], c["batch"]
    r = np.random.default_rng(5000 + c["i"])
    # stored shapes: A is M x K (op_a = N) or K x M; B is K x N (op_b = N) or N x K
    ar, acn = (K, M) if op_a else (M, K)
    br, bcn = (N, K) if op_b else (K, N)
    lda, ldb, ldc = acn + c["pa"], bcn + c["pb"], N + c["pc"]
    sa, sb, sc = ar * lda + 8 * (nb > 1), br * ldb + 8 * (nb > 1), M * ldc + 4 * (nb > 1)
    A = _mats(r, nb, sa, ar, acn, lda, ab, 1.0)
    B = _mats(r, nb, sb, br, bcn, ldb, ab, 0.05)
    C0 = _mats(r, nb, sc, M, N, ldc, ct, 1.0)
    Cin = _mats(r, nb, sc, M, N, ldc, ct, 1.0) if c["cin"] else None
    bias = (r.standard_normal(N) * 0.5).astype(np.float32) if c["bias"] else None
    gpu_c = C0.copy()
    if c["beta"] == 0.0:   # never read: NaN everywhere
        gpu_c[:] = NAN[ct]

    def dev(x, t):
        x = np.ascontiguousarray(x)
        return torch.from_numpy(x.view(np.int16) if x.dtype == np.uint16 else x).view(TD[t]).to("cuda:0")
    dA, dB, dC = dev(A, ab), dev(B, ab), dev(gpu_c, ct)
    dCin = dev(Cin, ct) if Cin is not None else None
    dBias = torch.from_numpy(bias).to("cuda:0") if bias is not None else None
    st = torch.cuda.current_stream().cuda_stream
    vk.gemm_ex_async(DT[ab], DT[ct], op_a, op_b, M, N, K, c["alpha"], dA.data_ptr(), lda, dB.data_ptr(), ldb,
                     c["beta"], dC.data_ptr(), ldc, batch=nb, stride_a=sa if nb > 1 else 0,
                     stride_b=sb if nb > 1 else 0, stride_c=sc if nb > 1 else 0, split_k=c["split"],
                     c_in=dCin.data_ptr() if dCin is not None else None, ldc_in=ldc if dCin is not None else 0,
                     stride_c_in=sc if (dCin is not None and nb > 1) else 0,
                     bias=dBias.data_ptr() if dBias is not None else None, bias_type=vk.DT_F32, stream=st)
    torch.cuda.synchronize()
    got_all = dC.cpu()
    got_all = (got_all.view(torch.int16).numpy().view(np.uint16) if ct != "f32" else got_all.numpy())
    rows = oracle.sample_rows(M, 16) if M * N * K > 64 * 1024 * 1024 else None
    sel = np.arange(M) if rows is None else rows
    if ab == "f32" and ct == "f32":
        bound = f32_bound(K)
    elif ct == "bf16":
        bound = BF16_BOUND
    else:
        bound = F16_BOUND
    for b in range(nb):
        want = C0[b * sc: b * sc + M * ldc].copy()
        cin = Cin[b * sc: b * sc + M * ldc].copy() if Cin is not None else want.copy()
        oracle.ref_gemm_epi_rm(ab, ct, op_a, op_b, M, N, K, np.ascontiguousarray(A[b * sa:(b + 1) * sa]), lda,
                               np.ascontiguousarray(B[b * sb:(b + 1) * sb]), ldb, c["alpha"], c["beta"],
                               np.ascontiguousarray(cin), ldc, want, ldc, bias, rows=rows)
        got = got_all[b * sc: b * sc + M * ldc]
        g = BACK[ct](np.stack([got[m * ldc: m * ldc + N] for m in sel]))
        w = BACK[ct](np.stack([want[m * ldc: m * ldc + N] for m in sel]))
        assert np.all(np.isfinite(g)), f"batch {b}: non-finite output"
        err = normwise(g, w)
        assert err <= bound, f"batch {b}: normwise {err:.3g} > {bound:.3g}"
        # padding columns of C are never written
        if c["pc"] and M > 1:
            padv = got[ldc - c["pc"]: ldc]
            assert np.array_equal(padv.view(np.uint32 if ct == "f32" else np.uint16),
                                  gpu_c[b * sc + N: b * sc + ldc].view(np.uint32 if ct == "f32" else np.uint16))
