"""HIP graph capture (torch.cuda.graph) of engine calls that need no
partials: the blocked and pipelined tile kernels (64x64 and 128x128 tiles,
fp32, fp16, bf16 to fp32), the one-token GEMV and the staged skinny decode
kernel.  Their launches go into the graph as kernel nodes (no allocation, no
memset); the graph is then replayed several times with eager work and
synchronisations between the replays, and every replay must equal the eager
result bit for bit.  Calls whose plan splits K need a workspace for their
partials and are not captured here (a capturing stream gets none; the test
of captured split calls in test_gpu_workspace.py stays skipped with its
reason).  No reference counterpart: the reference's engine waited for its
queue on every call (src/vkblas.c:954-968), so it could not be captured.
"""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

# (ab, ct, op_a, op_b, M, N, K)
CASES = [("f16", "f16", 0, 1, 1024, 1024, 1024),    # 128x128 pipelined tiles
         ("f32", "f32", 0, 0, 512, 512, 512),       # 64x64 tiles
         ("bf16", "f32", 1, 0, 2048, 2048, 512),    # 128x128 tiles, MN-major A, fp32 C
         ("f16", "f16", 0, 1, 1, 4096, 4096),       # GEMV (one token)
         ("f16", "f16", 0, 1, 8, 4096, 4096)]       # staged skinny decode, no K split
TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _bits(t):
    torch.cuda.synchronize()
    return t.cpu().view(torch.int16 if t.element_size() == 2 else torch.int32).numpy().copy()


def test_graph_capture_calls_without_partials():
    import vkblas_amd as vk
    dt = {"f32": vk.DT_F32, "f16": vk.DT_F16, "bf16": vk.DT_BF16}
    r = np.random.default_rng(77)
    ops = []
    for ab, ct, op_a, op_b, M, N, K in CASES:
        lda = M if op_a else K
        ldb = K if op_b else N
        pl = vk.plan(dt[ab], dt[ct], op_a, op_b, M, N, K, lda, ldb, N)
        # checked before anything is captured: no call here may need partials
        assert pl.split == 1 and pl.path not in (vk.PATH_SPLITK, vk.PATH_TAIL), (M, N, K, pl.path, pl.split)
        A = torch.from_numpy((r.standard_normal(M * K) * 0.5).astype(np.float32)).to(TD[ab]).to("cuda:0")
        B = torch.from_numpy((r.standard_normal(K * N) * 0.05).astype(np.float32)).to(TD[ab]).to("cuda:0")
        ops.append((ab, ct, op_a, op_b, M, N, K, lda, ldb, A, B, pl.path))

    def launch(o, out, stream):
        ab, ct, op_a, op_b, M, N, K, lda, ldb, A, B, _ = o
        vk.gemm_async(dt[ab], dt[ct], op_a, op_b, M, N, K, 1.0, A.data_ptr(), lda, B.data_ptr(), ldb, 0.0,
                      out.data_ptr(), N, stream=stream)

    eager = []
    for o in ops:
        c = torch.full((o[4] * o[5],), float("nan"), dtype=TD[o[1]], device="cuda:0")
        launch(o, c, torch.cuda.current_stream().cuda_stream)
        assert vk.last_path() == o[11]
        eager.append(_bits(c))
    # oracle check of the eager results (the graph replays must equal them)
    from gpu_helpers import normwise, f32_bound, F16_BOUND
    for o, e in zip(ops, eager):
        ab, ct, op_a, op_b, M, N, K, lda, ldb, A, B, _ = o
        conv = {"f32": lambda x: x, "f16": oracle.f2h_rne, "bf16": oracle.f2bf_rne}[ab]
        a = conv(A.float().cpu().numpy())
        b = conv(B.float().cpu().numpy())
        rows = oracle.sample_rows(M, 12) if M > 64 else None
        want = np.zeros(M * N, np.float32 if ct == "f32" else np.uint16)
        oracle.ref_gemm_epi_rm(ab, ct, op_a, op_b, M, N, K, a, lda, b, ldb, 1.0, 0.0, want.copy(), N, want, N,
                               None, rows=rows)
        sel = np.arange(M) if rows is None else rows
        back = (lambda x: x.view(np.float32)) if ct == "f32" else oracle.h2f
        g = back(e.view(np.uint32 if ct == "f32" else np.uint16)).reshape(M, N)[sel]
        w = back(want).reshape(M, N)[sel]
        assert normwise(g, w) <= (f32_bound(K) if (ab, ct) == ("f32", "f32") else F16_BOUND)

    outs = [torch.full((o[4] * o[5],), float("nan"), dtype=TD[o[1]], device="cuda:0") for o in ops]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):   # warm-up on a side stream before the capture
        for o, c in zip(ops, outs):
            launch(o, c, side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    print("[case] graph capture: tile, GEMV and skinny calls", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for o, c in zip(ops, outs):
            launch(o, c, torch.cuda.current_stream().cuda_stream)
    scratch = torch.full((ops[0][4] * ops[0][5],), float("nan"), dtype=TD[ops[0][1]], device="cuda:0")
    for rep in range(4):
        for c in outs:
            c.fill_(float("nan"))
        torch.cuda.synchronize()
        print(f"[case] graph replay {rep}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        for k, (c, e) in enumerate(zip(outs, eager)):
            assert np.array_equal(_bits(c), e), (rep, CASES[k])
        launch(ops[0], scratch, torch.cuda.current_stream().cuda_stream)   # eager work between replays
        torch.cuda.synchronize()
        assert np.array_equal(_bits(scratch), eager[0])
