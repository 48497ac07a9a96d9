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
