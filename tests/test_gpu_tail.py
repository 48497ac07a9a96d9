"""The split-tail plan (VKBLAS_PATH_TAIL) against the CPU oracle.

When a GEMM's tiles fill W whole waves and a last wave at most half full,
the planner runs the rows of the first tile rows as tiles and the last tile
rows (tail_rows of C) as split-K with as many slices as fit in one wave,
pass 1 on the same pipelined tile, then the fixed-order reduce with the
epilogue.  Checked here on the rows around the head / tail boundary and a
sample of the others, all four layouts, beta == 0 with NaN in C, beta != 0
in place and with a separate C_in and a bias (applied once, by the reduce for
the tail rows and by the tile epilogue for the head), a ragged M, fp32, fp16
and bf16; bitwise reproducible run to run; the allocation-free entry point
(partials in the library's scratch array) gives the same bits.  The oracle is
oracle.ref_gemm_epi_rm; the row-major engine contract is the reference's
src/vkblas.h:21-26.  No reference counterpart for the plan itself (the
reference split K only for few output tiles, src/vkblas.c:2850-2867).
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
CONV = {"f32": lambda x: x.astype(np.float32), "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}
BACK = {"f32": lambda x: x.astype(np.float32), "f16": oracle.h2f, "bf16": oracle.bf2f}


def _u(seed, n):
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


def _dev(x: np.ndarray, t: str) -> torch.Tensor:
    if x.dtype == np.uint16:
        return torch.from_numpy(x.view(np.int16)).view(TORCH_DT[t]).to("cuda:0")
    return torch.from_numpy(x).to("cuda:0")


def _host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.cpu().view(torch.int16).numpy().view(np.uint16)
    return t.cpu().numpy()


def _bound(ab, ct, K):
    from gpu_helpers import f32_bound, F16_BOUND, BF16_BOUND
    if ct == "bf16":
        return BF16_BOUND
    if ct == "f16" or ab != "f32":
        return F16_BOUND
    return f32_bound(K)


# (ab, ct, M, N, K): fp32 on 128x128 tiles (24 x 23 tiles: 1 wave of 512 + 40),
# fp32 with a ragged M (24 x 24 tiles, the last row partial), 16-bit on
# 256x256 tiles (18 x 16: 1 wave of 256 + 32)
SHAPES = [("f32", "f32", 3072, 2944, 2048), ("f32", "f32", 3000, 3072, 1024),
          ("f16", "f16", 4608, 4096, 2048), ("bf16", "f32", 4608, 4096, 2048)]
EPI = {"beta0": (0.0, False, None), "beta-inplace-bias": (0.5, False, "f32"), "cin-bias": (-0.75, True, "bf16")}


def run_tail(ab, ct, op_a, op_b, M, N, K, epi, noalloc=False):
    import vkblas_amd as vk
    from gpu_helpers import normwise
    beta, sep, bias_t = EPI[epi]
    dt = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    print(f"[case] tail {ab}>{ct} op={op_a}{op_b} {M}x{N}x{K} {epi} noalloc={noalloc}", flush=True)
    lda = M if op_a else K
    ldb = K if op_b else N
    ldc = N
    ldci = N + 8
    pl = vk.plan(dt[ab], dt[ct], op_a, op_b, M, N, K, lda, ldb, ldc)
    assert pl.path == vk.PATH_TAIL and pl.split >= 2 and 0 < pl.tail_rows < M, (pl.path, pl.split, pl.tail_rows)
    head = M - pl.tail_rows
    a = CONV[ab](_u(M + N + K + op_a, lda * (K if op_a else M)))
    b = CONV[ab](_u(3 * M + N + op_b, ldb * (N if op_b else K)))
    cin = CONV[ct](_u(7, ldci * M)) if sep else None
    d0 = CONV[ct](_u(9, ldc * M))
    if beta == 0.0:
        d0 = CONV[ct](np.full(ldc * M, np.nan, np.float32))
    bias = None if bias_t is None else CONV[bias_t](_u(11, N))
    rows = np.unique(np.concatenate([oracle.sample_rows(M, 12),
                                     np.array([0, head - 2, head - 1, head, head + 1, M - 2, M - 1], np.int32)]))
    rows = rows.astype(np.int32)
    want = d0.copy()
    oracle.ref_gemm_epi_rm(ab, ct, op_a, op_b, M, N, K, a, lda, b, ldb, 0.5 if beta else 1.25, beta,
                           cin.copy() if sep else want.copy(), ldci if sep else ldc, want, ldc,
                           None if bias is None else BACK[bias_t](bias), rows=rows)
    alpha = 0.5 if beta else 1.25
    dA, dB = _dev(a, ab), _dev(b, ab)
    dCin = _dev(cin, ct) if sep else None
    dBias = _dev(bias, bias_t) if bias is not None else None
    outs = []
    for rep in range(2):
        dD = _dev(d0, ct)
        if noalloc:
            assert not sep and bias is None
            vk.gemm_noalloc_async(dt[ab], dt[ct], op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb,
                                  beta, dD.data_ptr(), ldc)
        else:
            vk.gemm_ex_async(dt[ab], dt[ct], op_a, op_b, M, N, K, alpha, dA.data_ptr(), lda, dB.data_ptr(), ldb, beta,
                             dD.data_ptr(), ldc, c_in=dCin.data_ptr() if sep else None, ldc_in=ldci if sep else 0,
                             bias=dBias.data_ptr() if dBias is not None else None,
                             bias_type=dt[bias_t] if bias_t else vk.DT_F32)
        assert vk.last_path() == vk.PATH_TAIL
        outs.append(_host(dD))
    assert np.array_equal(outs[0].view(np.uint8), outs[1].view(np.uint8)), "not reproducible run to run"
    g = BACK[ct](outs[0]).reshape(M, ldc)[rows, :N].astype(np.float64)
    w = BACK[ct](want).reshape(M, ldc)[rows, :N].astype(np.float64)
    assert np.all(np.isfinite(g))
    assert normwise(g, w) <= _bound(ab, ct, K)
    # every row of C written (a NaN-filled C leaves no NaN behind)
    if beta == 0.0:
        assert np.all(np.isfinite(BACK[ct](outs[0])))
    return outs[0]


@pytest.mark.parametrize("epi", list(EPI))
@pytest.mark.parametrize("op_a,op_b", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s[0]}>{s[1]}-{s[2]}x{s[3]}x{s[4]}" for s in SHAPES])
def test_tail_plan(shape, op_a, op_b, epi):
    ab, ct, M, N, K = shape
    run_tail(ab, ct, op_a, op_b, M, N, K, epi)


@pytest.mark.parametrize("shape", [SHAPES[0], SHAPES[2]], ids=["f32", "f16"])
def test_tail_noalloc_same_bits(shape):
    """vkblas_gemm_noalloc_async runs the same plan with the tail's partials
    in the scratch array: the same bits as vkblas_gemm_async"""
    ab, ct, M, N, K = shape
    a = run_tail(ab, ct, 0, 1, M, N, K, "beta0")
    b = run_tail(ab, ct, 0, 1, M, N, K, "beta0", noalloc=True)
    assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
