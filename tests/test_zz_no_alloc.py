"""vkblas_gemm_noalloc_async against vkblas_gemm_async, through the C ABI.

The allocation-free entry point runs the same plan and kernels with the
split-K / split-decode partials in the library's per-device scratch array.
Two calls in a row per path, the second on a smaller input (the array then
holds the first call's partials): each result equals vkblas_gemm_async's
bit for bit (both sum the partials in the same fixed order) and the CPU
oracle within the parity bars.  A call whose partials exceed the array is
rejected before launching (C untouched).  No reference counterpart: the
entry point exists for callers that cannot allocate.
"""
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


def _dev(x: np.ndarray, half: bool) -> torch.Tensor:
    if half:
        return torch.from_numpy(oracle.f2h_rne(x).view(np.int16)).view(torch.float16).to("cuda:0")
    return torch.from_numpy(x).to("cuda:0")


# (label, ab, op_a, op_b, M, N, K, expected path): the second of each pair is smaller
CASES = [
    ("splitk-f16", "f16", 0, 0, 256, 256, 65536, "splitk"),
    ("splitk-f16", "f16", 0, 0, 256, 128, 8192, "splitk"),
    ("splitk-f32", "f32", 0, 0, 256, 256, 65536, "splitk"),
    ("splitk-f32", "f32", 1, 1, 128, 256, 16384, "splitk"),
    ("decode-f16", "f16", 0, 1, 24, 8192, 8192, "skinny"),
    ("decode-f16", "f16", 0, 1, 20, 4096, 4096, "skinny"),
    ("tile-f16", "f16", 0, 0, 512, 512, 512, "tile"),
    ("tile-f16", "f16", 1, 0, 256, 256, 256, "tile"),
    # weight K x N: the 16-bit K x N decode kernel's K split (8 and 15 slices)
    ("decode-kn-f16", "f16", 0, 0, 16, 8192, 8192, "skinny"),
    ("decode-kn-f16", "f16", 0, 0, 33, 2048, 8200, "skinny"),
]


@pytest.mark.parametrize("pair", [0, 1, 2, 3, 4],
                         ids=["splitk-f16", "splitk-f32", "decode-f16", "tile-f16", "decode-kn-f16"])
def test_noalloc_matches_gemm_async(pair):
    import vkblas_amd as vk
    from gpu_helpers import normwise, f32_bound, F16_BOUND
    for case in CASES[2 * pair: 2 * pair + 2]:
        label, ab, op_a, op_b, M, N, K, path = case
        print(f"[case] noalloc {case}", flush=True)
        half = ab == "f16"
        dt = vk.DT_F16 if half else vk.DT_F32
        lda = M if op_a else K
        ldb = K if op_b else N
        a = _u(M + 7 * N + K, lda * (K if op_a else M))
        b = (_u(3 * M + N + 5 * K, ldb * (N if op_b else K)) * (0.05 if path == "skinny" else 1.0)).astype(np.float32)
        dA, dB = _dev(a, half), _dev(b, half)
        tdt = torch.float16 if half else torch.float32
        c_ref = torch.full((M * N,), float("nan"), dtype=tdt, device="cuda:0")
        c_na = torch.full((M * N,), float("nan"), dtype=tdt, device="cuda:0")
        vk.gemm_async(dt, dt, op_a, op_b, M, N, K, 1.0, dA.data_ptr(), lda, dB.data_ptr(), ldb, 0.0, c_ref.data_ptr(), N)
        p_ref = vk.last_path()
        vk.gemm_noalloc_async(dt, dt, op_a, op_b, M, N, K, 1.0, dA.data_ptr(), lda, dB.data_ptr(), ldb, 0.0,
                              c_na.data_ptr(), N)
        assert vk.last_path() == p_ref
        if path == "splitk":
            assert p_ref == vk.PATH_SPLITK
        elif path == "skinny":
            assert p_ref == vk.PATH_SKINNY
        got = _bits(c_na)
        assert np.array_equal(got, _bits(c_ref)), f"{case}: noalloc result differs from vkblas_gemm_async"
        rows = oracle.sample_rows(M, 12) if M > 64 else None
        sel = np.arange(M) if rows is None else rows
        if half:
            ref = np.zeros(M * N, np.uint16)
            oracle.ref_gemm_f16_rm(op_a, op_b, M, N, K, oracle.f2h_rne(a), lda, oracle.f2h_rne(b), ldb, 1.0, 0.0,
                                   ref, N, rows=rows)
            g = oracle.h2f(got.view(np.uint16).reshape(M, N)[sel])
            r = oracle.h2f(ref.reshape(M, N)[sel])
            assert normwise(g, r) <= F16_BOUND
        else:
            ref = np.zeros(M * N, np.float32)
            oracle.ref_gemm_f32_rm(op_a, op_b, M, N, K, a, lda, b, ldb, 1.0, 0.0, ref, N, rows=rows)
            g = got.view(np.float32).reshape(M, N)[sel]
            r = ref.reshape(M, N)[sel]
            assert normwise(g, r) <= f32_bound(K)


def test_noalloc_rejects_partials_beyond_scratch():
    import vkblas_amd as vk
    print("[case] noalloc rejects oversized partials", flush=True)
    M = N = 1024
    K = 8192
    assert 128 * M * N * 4 > vk.noalloc_scratch_bytes()
    dA = torch.zeros(M * K, device="cuda:0")
    dB = torch.zeros(K * N, device="cuda:0")
    dC = torch.full((M * N,), 7.0, device="cuda:0")
    st = vk.gemm_noalloc_async(vk.DT_F32, vk.DT_F32, 0, 0, M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 0.0,
                               dC.data_ptr(), N, split_k=128, check=False)
    assert st == vk.ERR_PARAM
    torch.cuda.synchronize()
    assert torch.all(dC == 7.0)
    # the same call with partials that fit runs
    vk.gemm_noalloc_async(vk.DT_F32, vk.DT_F32, 0, 0, M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 0.0,
                          dC.data_ptr(), N, split_k=8)
    torch.cuda.synchronize()
    assert torch.all(dC == 0.0)


def test_noalloc_divided_slices_match_gemm_async():
    """A caller's split run with each K slice divided among four workgroups
    (their arrival counters at the start of the scratch array, cleared on the
    device's first no-alloc call): the same bits as vkblas_gemm_async, on two
    calls in a row, the second smaller."""
    import vkblas_amd as vk
    from gpu_helpers import to_host
    print("[case] noalloc divided K slices", flush=True)
    for M, N, K, split in ((256, 256, 16384, 4), (128, 256, 8192, 9)):
        pl = vk.plan(vk.DT_F32, vk.DT_F32, 0, 0, M, N, K, K, N, N, split_k=split)
        assert (pl.path, pl.split, pl.tile) == (vk.PATH_SPLITK, split, 4), (M, N, K, pl.tile)
        a = np.random.default_rng(M + split).uniform(-1, 1, M * K).astype(np.float32)
        b = np.random.default_rng(N + split).uniform(-1, 1, K * N).astype(np.float32)
        dA, dB = torch.from_numpy(a).to("cuda:0"), torch.from_numpy(b).to("cuda:0")
        c_ref = torch.full((M * N,), float("nan"), device="cuda:0")
        c_na = torch.full((M * N,), float("nan"), device="cuda:0")
        vk.gemm_async(vk.DT_F32, vk.DT_F32, 0, 0, M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 0.0,
                      c_ref.data_ptr(), N, split_k=split)
        vk.gemm_noalloc_async(vk.DT_F32, vk.DT_F32, 0, 0, M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 0.0,
                              c_na.data_ptr(), N, split_k=split)
        assert vk.last_kernel() == vk.KERNEL_WAVEK
        assert np.array_equal(to_host(c_na).view(np.uint32), to_host(c_ref).view(np.uint32)), (M, N, K, split)
