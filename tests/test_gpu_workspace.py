"""The split-K / decode partials workspace under the ways callers drive it.

  * HIP graph capture (torch.cuda.graph): a split-K call and a split decode
    call captured, the graph replayed several times with eager work and
    synchronisations between the replays; every replay equals the eager
    result bit for bit and the oracle within the parity bars.  (Skipped: see
    its marker.)
  * hipStreamPerThread (handle value 2, a different stream in every thread).
  * Two host threads launching split-K calls on ONE stream at once: a call
    keeps its stream's buffer until its reduce is queued, so every result
    equals the call made alone, bit for bit.
  * vkblas_workspace_release, then more calls; and from a third thread while
    two threads issue split-K calls that grow their buffers.
  * Four streams fed at once by four threads with a mix of calls that need
    partials (split-K, divided K slices with their arrival counters, split
    decodes in both weight layouts, the split tail).

The split-K contract is the reference's two-pass scheme (src/vkblas.c:1873-1984,
src/shaders/splitk_reduce_f32.comp:15-24); its partials were grow-only
(src/vkblas.c:1889-1914).
"""
import threading

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _u(seed, n):
    return np.random.default_rng(seed).uniform(-1.0, 1.0, n).astype(np.float32)


def _bits(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().view(torch.int16 if t.element_size() == 2 else torch.int32).numpy().copy()


def _f16(x: np.ndarray, dev="cuda:0") -> torch.Tensor:
    return torch.from_numpy(oracle.f2h_rne(x).view(np.int16)).view(torch.float16).to(dev)


def _splitk_case():
    """fp16 M = N = 256, K = 16384: the planner's split-K (128x128 tiles)."""
    M = N = 256
    K = 16384
    a, b = _u(901, M * K), _u(902, K * N)
    return M, N, K, a, b


def _decode_case():
    """fp16 decode, 24 tokens x 8192 x 4096: the planner splits K (partials)."""
    M, N, K = 24, 8192, 4096
    x, w = _u(903, M * K), (_u(904, N * K) * 0.05).astype(np.float32)
    return M, N, K, x, w


def _run_splitk(vk, dA, dB, dC, M, N, K, stream):
    vk.gemm_async(vk.DT_F16, vk.DT_F16, vk.OP_N, vk.OP_N, M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 0.0,
                  dC.data_ptr(), N, stream=stream)


def _run_decode(vk, dX, dW, dC, M, N, K, stream):
    vk.gemm_async(vk.DT_F16, vk.DT_F16, vk.OP_N, vk.OP_T, M, N, K, 1.0, dX.data_ptr(), K, dW.data_ptr(), K, 0.0,
                  dC.data_ptr(), N, stream=stream)


def _check_f16(got_bits, M, N, K, a, lda, b, ldb, op_a, op_b):
    from gpu_helpers import normwise, F16_BOUND
    ref = np.zeros(M * N, np.uint16)
    ha, hb = oracle.f2h_rne(a), oracle.f2h_rne(b)
    rows = oracle.sample_rows(M, 12) if M > 64 else None
    oracle.ref_gemm_f16_rm(op_a, op_b, M, N, K, ha, lda, hb, ldb, 1.0, 0.0, ref, N, rows=rows)
    sel = np.arange(M) if rows is None else rows
    g = oracle.h2f(got_bits.view(np.uint16).reshape(M, N)[sel])
    r = oracle.h2f(ref.reshape(M, N)[sel])
    assert normwise(g, r) <= F16_BOUND


@pytest.mark.skip(reason="faulted the GPU box in the run that introduced it (allocation of the partials inside "
                         "the capture, graph-owned memory); that code is removed and captured calls needing partials "
                         "now decline (the cause was not shown, so this case stays off the GPU)")
def test_graph_capture_splitk_and_decode():
    import vkblas_amd as vk
    print("[case] graph capture: split-K + split decode", flush=True)
    M, N, K, a, b = _splitk_case()
    dM, dN, dK, x, w = _decode_case()
    pl = vk.plan(vk.DT_F16, vk.DT_F16, vk.OP_N, vk.OP_N, M, N, K, K, N, N)
    assert pl.path == vk.PATH_SPLITK and pl.split > 1
    pd = vk.plan(vk.DT_F16, vk.DT_F16, vk.OP_N, vk.OP_T, dM, dN, dK, dK, dK, dN)
    assert pd.path == vk.PATH_SKINNY and pd.split > 1
    dA, dB = _f16(a), _f16(b)
    dX, dW = _f16(x), _f16(w)
    # eager results first
    eC = torch.full((M * N,), float("nan"), dtype=torch.float16, device="cuda:0")
    eY = torch.full((dM * dN,), float("nan"), dtype=torch.float16, device="cuda:0")
    cur = torch.cuda.current_stream().cuda_stream
    _run_splitk(vk, dA, dB, eC, M, N, K, cur)
    _run_decode(vk, dX, dW, eY, dM, dN, dK, cur)
    e_c, e_y = _bits(eC), _bits(eY)
    _check_f16(e_c, M, N, K, a, K, b, N, 0, 0)
    _check_f16(e_y, dM, dN, dK, x, dK, w, dK, 0, 1)

    gC = torch.full((M * N,), float("nan"), dtype=torch.float16, device="cuda:0")
    gY = torch.full((dM * dN,), float("nan"), dtype=torch.float16, device="cuda:0")
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            s = torch.cuda.current_stream().cuda_stream
            _run_splitk(vk, dA, dB, gC, M, N, K, s)
            _run_decode(vk, dX, dW, gY, dM, dN, dK, s)
    torch.cuda.synchronize()
    other = torch.full((M * N,), 0.0, dtype=torch.float16, device="cuda:0")
    for rep in range(3):
        gC.fill_(float("nan"))
        gY.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_bits(gC), e_c), f"replay {rep}: split-K differs from the eager call"
        assert np.array_equal(_bits(gY), e_y), f"replay {rep}: decode differs from the eager call"
        # eager calls on the same shapes between replays (they use the cached
        # per-stream workspace, the replays their own)
        _run_splitk(vk, dA, dB, other, M, N, K, cur)
        assert np.array_equal(_bits(other), e_c)


def test_per_thread_default_stream():
    """hipStreamPerThread (handle 2): each thread's calls run on its own
    per-thread stream; partials are never shared through one slot."""
    import vkblas_amd as vk
    print("[case] hipStreamPerThread split-K from two threads", flush=True)
    M, N, K, a, b = _splitk_case()
    dA, dB = _f16(a), _f16(b)
    ref = torch.full((M * N,), float("nan"), dtype=torch.float16, device="cuda:0")
    _run_splitk(vk, dA, dB, ref, M, N, K, None)
    want = _bits(ref)
    outs = [[torch.full((M * N,), float("nan"), dtype=torch.float16, device="cuda:0") for _ in range(4)]
            for _ in range(2)]
    torch.cuda.synchronize()
    errors = []

    def worker(t):
        try:
            for i in range(4):
                _run_splitk(vk, dA, dB, outs[t][i], M, N, K, 2)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    ths = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    assert not errors
    torch.cuda.synchronize()   # a device-wide wait: covers every thread's per-thread stream
    for t in range(2):
        for i in range(4):
            assert np.array_equal(_bits(outs[t][i]), want)


def test_two_threads_one_stream():
    """Two threads issue split-K calls on the SAME stream at once, with
    different operands and growing splits: each call's pass 1 and reduce
    stay paired on the stream's buffer."""
    import vkblas_amd as vk
    print("[case] two threads, one stream, split-K", flush=True)
    M, N, K = 128, 128, 16384
    A = [torch.from_numpy(_u(920 + t, M * K)).to("cuda:0") for t in range(2)]
    B = [torch.from_numpy(_u(930 + t, K * N)).to("cuda:0") for t in range(2)]
    splits = (4, 16, 64)
    alone = {}
    for t in range(2):
        for sp in splits:
            c = torch.empty(M * N, dtype=torch.float32, device="cuda:0")
            vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, vk.OP_N, M, N, K, 1.0, A[t].data_ptr(), K, B[t].data_ptr(),
                          N, 0.0, c.data_ptr(), N, split_k=sp)
            alone[t, sp] = _bits(c)
    st = torch.cuda.Stream()
    calls = 12
    outs = [[torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda:0") for _ in range(calls)]
            for _ in range(2)]
    torch.cuda.synchronize()
    errors = []

    def worker(t):
        try:
            for i in range(calls):
                vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, vk.OP_N, M, N, K, 1.0, A[t].data_ptr(), K,
                              B[t].data_ptr(), N, 0.0, outs[t][i].data_ptr(), N, split_k=splits[i % 3],
                              stream=st.cuda_stream)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    ths = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    assert not errors
    torch.cuda.synchronize()
    for t in range(2):
        for i in range(calls):
            assert np.array_equal(_bits(outs[t][i]), alone[t, splits[i % 3]])


def test_workspace_release_then_reuse():
    import vkblas_amd as vk
    print("[case] workspace release", flush=True)
    M, N, K, a, b = _splitk_case()
    dA, dB = _f16(a), _f16(b)
    c0 = torch.full((M * N,), float("nan"), dtype=torch.float16, device="cuda:0")
    _run_splitk(vk, dA, dB, c0, M, N, K, None)
    want = _bits(c0)
    vk.workspace_release()
    c1 = torch.full((M * N,), float("nan"), dtype=torch.float16, device="cuda:0")
    _run_splitk(vk, dA, dB, c1, M, N, K, None)
    assert np.array_equal(_bits(c1), want)
    vk.workspace_release()
    vk.workspace_release()


def test_workspace_release_during_calls():
    """vkblas_workspace_release from one thread while two others issue
    split-K calls whose partials grow their streams' buffers: the release
    takes each slot's lock before the pool lock, as the calls do, so every
    thread finishes (bounded joins) and every result equals the call made
    alone."""
    import vkblas_amd as vk
    print("[case] workspace release during split-K calls", flush=True)
    M, N, K = 128, 128, 16384
    A = torch.from_numpy(_u(940, M * K)).to("cuda:0")
    B = torch.from_numpy(_u(941, K * N)).to("cuda:0")
    splits = (4, 16, 64)
    alone = {}
    for sp in splits:
        c = torch.empty(M * N, dtype=torch.float32, device="cuda:0")
        vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, vk.OP_N, M, N, K, 1.0, A.data_ptr(), K, B.data_ptr(), N, 0.0,
                      c.data_ptr(), N, split_k=sp)
        alone[sp] = _bits(c)
    calls = 18
    streams = [torch.cuda.Stream() for _ in range(2)]
    outs = [[torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda:0") for _ in range(calls)]
            for _ in range(2)]
    torch.cuda.synchronize()
    errors = []
    done = threading.Event()

    def worker(t):
        try:
            for i in range(calls):
                vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, vk.OP_N, M, N, K, 1.0, A.data_ptr(), K, B.data_ptr(),
                              N, 0.0, outs[t][i].data_ptr(), N, split_k=splits[i % 3],
                              stream=streams[t].cuda_stream)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    def releaser():
        try:
            while not done.is_set():
                vk.workspace_release()
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    rel = threading.Thread(target=releaser, daemon=True)
    ths = [threading.Thread(target=worker, args=(t,), daemon=True) for t in range(2)]
    rel.start()
    for th in ths:
        th.start()
    for th in ths:
        th.join(timeout=60)
    done.set()
    rel.join(timeout=60)
    assert not any(th.is_alive() for th in ths + [rel]), "a thread did not finish"
    assert not errors
    torch.cuda.synchronize()
    for t in range(2):
        for i in range(calls):
            assert np.array_equal(_bits(outs[t][i]), alone[splits[i % 3]])
    vk.workspace_release()


CHILD_NO_ROOM = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1])
import oracle, vkblas_amd as vk
from gpu_helpers import normwise, f32_bound
M = N = 1024; K = 8192
rng = np.random.default_rng(5)
a = rng.uniform(-1, 1, M * K).astype(np.float32); b = rng.uniform(-1, 1, K * N).astype(np.float32)
dA, dB = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
pl = vk.plan(vk.DT_F32, vk.DT_F32, 0, 0, M, N, K, K, N, N)
assert pl.path == vk.PATH_SPLITK and pl.split == 128, (pl.path, pl.split)
assert pl.split * M * N * 4 > vk.noalloc_scratch_bytes()
rows = oracle.sample_rows(M, 12)
ref = np.zeros(M * N, np.float32)
oracle.ref_gemm_f32_rm(0, 0, M, N, K, a, K, b, N, 1.0, 0.0, ref, N, rows=rows)
for name in ("noalloc", "async"):
    dC = torch.full((M * N,), float("nan"), device="cuda:0")
    fn = vk.gemm_noalloc_async if name == "noalloc" else vk.gemm_async
    fn(vk.DT_F32, vk.DT_F32, 0, 0, M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 0.0, dC.data_ptr(), N)
    path = vk.last_path()
    # the scratch has no room for 128 slices: the heuristic split falls back
    # to the plan without a split; the workspace path keeps the split
    assert path == (vk.PATH_TILE128 if name == "noalloc" else vk.PATH_SPLITK), (name, path)
    got = dC.cpu().numpy().reshape(M, N)[rows]
    assert normwise(got, ref.reshape(M, N)[rows]) <= f32_bound(K), name
print("NO ROOM OK")
"""


def test_heuristic_split_without_room_runs_unsplit(tmp_path):
    """A planner-chosen split (here VKBLAS_SPLITK=128, which sets the
    heuristic's split) whose partials exceed the no-alloc scratch runs
    without a split instead of failing; a caller's split_k > 1 is still
    rejected (test_zz_no_alloc).  Runs in a child process: VKBLAS_SPLITK is
    read once per process."""
    import os
    import subprocess
    import sys
    print("[case] heuristic split without room for the partials", flush=True)
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, VKBLAS_SPLITK="128", PYTHONPATH=os.path.join(repo, "tests") + os.pathsep + repo)
    r = subprocess.run([sys.executable, "-c", CHILD_NO_ROOM, repo], env=env, capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and "NO ROOM OK" in r.stdout, f"rc={r.returncode}\n{r.stdout[-3000:]}\n{r.stderr[-3000:]}"


def test_four_streams_mixed_calls_at_once():
    """Four streams, each fed by its own host thread with a different mix of
    calls that need partials (planner split-K, a caller's split 4 with K
    slices divided among workgroups and their arrival counters, a split
    decode, the split tail): every stream keeps its own workspace, so every
    result equals the same call made alone, bit for bit."""
    import vkblas_amd as vk
    print("[case] four streams, mixed partial-using calls", flush=True)
    r = np.random.default_rng(950)
    h16 = lambda n, s=1.0: torch.from_numpy(oracle.f2h_rne((r.standard_normal(n) * s).astype(np.float32))
                                            .view(np.int16)).view(torch.float16).to("cuda:0")
    # (label, ab, ct, op_a, op_b, M, N, K, split_k, operand scale of B)
    calls = [("splitk", vk.DT_F16, vk.DT_F16, 0, 0, 256, 256, 16384, 0, 1.0),
             ("divided", vk.DT_F16, vk.DT_F32, 0, 0, 256, 256, 16384, 4, 1.0),
             ("decode", vk.DT_F16, vk.DT_F16, 0, 1, 24, 8192, 4096, 0, 0.05),
             ("decode_kn", vk.DT_F16, vk.DT_F16, 0, 0, 16, 8192, 8192, 0, 0.05),
             ("tail", vk.DT_F16, vk.DT_F16, 0, 0, 4608, 4096, 2048, 0, 1.0)]
    ops = []
    for label, ab, ct, op_a, op_b, M, N, K, sp, sc in calls:
        lda = M if op_a else K
        ldb = K if op_b else N
        A, B = h16(M * K), h16(K * N, sc)
        pl = vk.plan(ab, ct, op_a, op_b, M, N, K, lda, ldb, N, split_k=sp)
        assert pl.split > 1 or pl.path == vk.PATH_TAIL, (label, pl.path, pl.split)
        ops.append((label, ab, ct, op_a, op_b, M, N, K, sp, lda, ldb, A, B))

    def launch(o, out, stream):
        label, ab, ct, op_a, op_b, M, N, K, sp, lda, ldb, A, B = o
        vk.gemm_async(ab, ct, op_a, op_b, M, N, K, 1.0, A.data_ptr(), lda, B.data_ptr(), ldb, 0.0, out.data_ptr(), N,
                      split_k=sp, stream=stream)

    def new_out(o):
        return torch.full((o[5] * o[6],), float("nan"), dtype=torch.float32 if o[2] == vk.DT_F32 else torch.float16,
                          device="cuda:0")
    alone = []
    for o in ops:
        c = new_out(o)
        launch(o, c, None)
        alone.append(_bits(c))
    streams = [torch.cuda.Stream() for _ in range(4)]
    rounds = 3
    outs = [[[new_out(o) for o in ops] for _ in range(rounds)] for _ in range(4)]
    torch.cuda.synchronize()
    errors = []

    def worker(s):
        try:
            for rd in range(rounds):
                for j in range(len(ops)):
                    k = (j + s + rd) % len(ops)       # each stream its own order
                    launch(ops[k], outs[s][rd][k], streams[s].cuda_stream)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    ths = [threading.Thread(target=worker, args=(s,)) for s in range(4)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    assert not errors, errors
    torch.cuda.synchronize()
    for s in range(4):
        for rd in range(rounds):
            for k in range(len(ops)):
                assert np.array_equal(_bits(outs[s][rd][k]), alone[k]), (s, rd, ops[k][0])
