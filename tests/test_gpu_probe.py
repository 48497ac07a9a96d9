"""vkblas_mfma_probe (the bench-only MFMA-rate measurement bench.py reports): its sums
are exact for constant operands, so the test checks the kernel issues every
MFMA it claims to."""
import pytest

torch = pytest.importorskip("torch")

from vkblas_amd import bench_probe as probe

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("blocks,iters", [(1, 1), (3, 7), (256, 40)])
def test_mfma_probe_exact_sums(bf16, blocks, iters):
    dt = torch.bfloat16 if bf16 else torch.float16
    out = torch.full((blocks * 256,), float("nan"), device="cuda:0")
    ones = torch.ones(12 * 64 * 8, device="cuda:0", dtype=dt)
    probe.mfma_probe(bf16, ones.data_ptr(), out.data_ptr(), blocks, iters)
    torch.cuda.synchronize()
    # every accumulator element gains 32 (one 32-long dot product of ones) per
    # round; a thread sums 32 tiles x 4 elements
    assert torch.all(out == 32.0 * 4 * 32 * iters)
    zeros = torch.zeros_like(ones)
    probe.mfma_probe(bf16, zeros.data_ptr(), out.data_ptr(), blocks, iters)
    torch.cuda.synchronize()
    assert torch.all(out == 0.0)


def test_mfma_probe_rejects_bad_arguments():
    ops = torch.zeros(12 * 64 * 8, device="cuda:0", dtype=torch.float16)
    out = torch.zeros(256, device="cuda:0")
    with pytest.raises(RuntimeError):
        probe.mfma_probe(False, ops.data_ptr(), out.data_ptr(), 0, 1)
    with pytest.raises(RuntimeError):
        probe.mfma_probe(False, ops.data_ptr() + 2, out.data_ptr(), 1, 1)


def _last_step_sums(a16, n, blocks, row_bytes):
    """Expected copy_probe checksums: per workgroup b, the wrapping 32-bit sum
    of the words of its tile's last K step (A rows m0 .. m0 + 255 and B rows
    n0 .. n0 + 255, the last row_bytes of each row)."""
    import numpy as np
    A, B = a16
    tiles = n // 256
    ks = row_bytes // 2
    out = []
    for b in range(blocks):
        # the GEMM kernel's tile order: XCD runs, then groups of 4 tile rows
        t = (b & 7) * (blocks >> 3) + (b >> 3) if blocks % 8 == 0 else b
        group, tin = t // (4 * tiles), t % (4 * tiles)
        gm = min(tiles - 4 * group, 4)
        m0, n0 = (4 * group + tin % gm) * 256, (tin // gm) * 256
        s = 0
        for M, r0 in ((A, m0), (B, n0)):
            w = np.ascontiguousarray(M[r0:r0 + 256, n - ks:]).view(np.uint32)
            s += int(w.astype(np.uint64).sum())
        out.append(s & 0xFFFFFFFF)
    return out


@pytest.mark.parametrize("steps_in_flight", [1, 2])
@pytest.mark.parametrize("row_bytes", [128, 64])
@pytest.mark.parametrize("n,blocks", [(768, 9), (1024, 16), (1280, 24)])
def test_copy_probe_lands_the_last_step(steps_in_flight, row_bytes, n, blocks):
    """vkblas_copy_probe (the bench-only L2 -> LDS copy-rate measurement):
    each workgroup's last LDS stage holds exactly its tile's last K step of A
    and B rows, so the copies land where the kernel claims (grids of 9 tiles,
    16 and 24 of 25 tiles: the XCD-run tile order)."""
    import numpy as np
    g = torch.Generator(device="cpu").manual_seed(5)
    A = torch.randint(0, 65536, (n, n), generator=g, dtype=torch.int32).to(torch.int16)
    B = torch.randint(0, 65536, (n, n), generator=g, dtype=torch.int32).to(torch.int16)
    dA, dB = A.to("cuda:0"), B.to("cuda:0")
    out = torch.zeros(blocks, device="cuda:0", dtype=torch.int32)
    probe.copy_probe(dA.data_ptr(), dB.data_ptr(), n, blocks, steps_in_flight, row_bytes, out.data_ptr())
    torch.cuda.synchronize()
    got = [v & 0xFFFFFFFF for v in out.cpu().tolist()]
    want = _last_step_sums((A.numpy().view(np.uint16), B.numpy().view(np.uint16)), n, blocks, row_bytes)
    assert got == want


def test_copy_probe_rejects_bad_arguments():
    a = torch.zeros(512 * 512, device="cuda:0", dtype=torch.float16)
    out = torch.zeros(16, device="cuda:0", dtype=torch.int32)
    for n, blocks, d, rb, off in ((500, 1, 1, 128, 0), (512, 5, 1, 128, 0), (512, 0, 1, 128, 0),
                                  (512, 1, 3, 128, 0), (512, 1, 1, 96, 0), (512, 1, 1, 128, 2)):
        with pytest.raises(RuntimeError):
            probe.copy_probe(a.data_ptr() + off, a.data_ptr(), n, blocks, d, rb, out.data_ptr())
