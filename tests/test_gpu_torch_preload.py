"""PyTorch-ROCm with libvkblas_hipblas.so preloaded, the reference's main use
(reference README.md:56-70, test/test_torch.py): torch's matmul, bmm and
linear must reach this library's hipBLAS entry points and give the right
answers.  Each case runs in a child process started with the preload
environment of vkblas_amd.preload; VKBLAS_TRACE=1 makes the library log every
GEMM it takes, so the test can tell an intercepted call from one that went to
the real hipBLAS.  The child selects PyTorch's hipBLAS backend with
torch.backends.cuda.preferred_blas_library("cublas"), as a PyTorch user of the
library must on gfx950 (the default there is hipBLASLt).
"""
import json
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

CHILD = r"""
import json, torch
# the hipBLAS backend (PyTorch's default on gfx950 is hipBLASLt)
torch.backends.cuda.preferred_blas_library("cublas")
torch.manual_seed(0)
dev = "cuda:0"
out = {}
def rel(got, ref):
    got = got.double().cpu(); ref = ref.double().cpu()
    return float((got - ref).abs().max() / ref.abs().max())
# fp32 matmul (hipblasSgemm), all four layouts through transposed views
a = torch.rand(257, 129, device=dev) * 2 - 1
b = torch.rand(129, 65, device=dev) * 2 - 1
out["mm_nn"] = rel(a @ b, a.cpu().double() @ b.cpu().double())
at = (torch.rand(129, 257, device=dev) * 2 - 1)
out["mm_tn"] = rel(at.t() @ b, at.cpu().double().t() @ b.cpu().double())
bt = (torch.rand(65, 129, device=dev) * 2 - 1)
out["mm_nt"] = rel(a @ bt.t(), a.cpu().double() @ bt.cpu().double().t())
out["mm_tt"] = rel(at.t() @ bt.t(), at.cpu().double().t() @ bt.cpu().double().t())
# addmm with beta (alpha / beta epilogue)
c0 = torch.rand(257, 65, device=dev)
out["addmm"] = rel(torch.addmm(c0, a, b, beta=0.5, alpha=2.0),
                   0.5 * c0.cpu().double() + 2.0 * (a.cpu().double() @ b.cpu().double()))
# fp32 bmm (hipblasSgemmStridedBatched)
A = torch.rand(8, 64, 96, device=dev); B = torch.rand(8, 96, 48, device=dev)
out["bmm"] = rel(torch.bmm(A, B), torch.bmm(A.cpu().double(), B.cpu().double()))
# fp16 matmul (hipblasGemmEx 16F, fp32 accumulation)
h1 = (torch.randn(512, 1024, device=dev) / 32).half(); h2 = torch.randn(1024, 384, device=dev).half()
out["mm_f16"] = rel(h1 @ h2, h1.cpu().double() @ h2.cpu().double())
# fp16 decode linear: W (O, K) row-major = hipBLAS TA=T, the skinny path
W = (torch.randn(4096, 2048, device=dev) * 0.02).half(); x = torch.randn(4, 2048, device=dev).half()
out["linear_decode_f16"] = rel(torch.nn.functional.linear(x, W), x.cpu().double() @ W.cpu().double().t())
# bf16 matmul, bmm and linear (hipblasGemmEx / GemmStridedBatchedEx with 16BF data).
# A linear with a bias is left out: PyTorch computes that one with a fused
# bias epilogue in another library, not through hipBLAS / rocBLAS.
g1 = (torch.randn(384, 1024, device=dev) / 32).bfloat16(); g2 = torch.randn(1024, 640, device=dev).bfloat16()
out["mm_bf16"] = rel(g1 @ g2, g1.cpu().double() @ g2.cpu().double())
G1 = torch.randn(4, 128, 256, device=dev).bfloat16(); G2 = (torch.randn(4, 256, 96, device=dev) / 16).bfloat16()
out["bmm_bf16"] = rel(torch.bmm(G1, G2), torch.bmm(G1.cpu().double(), G2.cpu().double()))
Wb = (torch.randn(768, 512, device=dev) * 0.05).bfloat16(); xb = torch.randn(64, 512, device=dev).bfloat16()
out["linear_bf16"] = rel(torch.nn.functional.linear(xb, Wb), xb.cpu().double() @ Wb.cpu().double().t())
# bf16 decode linear (2 tokens): the skinny path
xd = torch.randn(2, 512, device=dev).bfloat16()
out["linear_decode_bf16"] = rel(torch.nn.functional.linear(xd, Wb), xd.cpu().double() @ Wb.cpu().double().t())
torch.cuda.synchronize()
print("RESULT " + json.dumps(out), flush=True)
"""

BOUNDS = {"mm_nn": 1e-5 * 129 ** 0.5, "mm_tn": 1e-5 * 129 ** 0.5, "mm_nt": 1e-5 * 129 ** 0.5,
          "mm_tt": 1e-5 * 129 ** 0.5, "addmm": 1e-5 * 129 ** 0.5, "bmm": 1e-5 * 96 ** 0.5,
          "mm_f16": 2e-3, "linear_decode_f16": 2e-3,
          # bf16 results: one rounding to bf16 (2^-8 relative) plus fp32 sums
          "mm_bf16": 8e-3, "bmm_bf16": 8e-3, "linear_bf16": 8e-3, "linear_decode_bf16": 8e-3}


def test_torch_ops_go_through_the_library():
    from vkblas_amd.preload import preload_env
    env = preload_env()
    env["VKBLAS_TRACE"] = "1"
    print("[case] torch under LD_PRELOAD", env["LD_PRELOAD"], flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    line = next(l for l in r.stdout.splitlines() if l.startswith("RESULT "))
    res = json.loads(line[len("RESULT "):])
    for k, bound in BOUNDS.items():
        assert res[k] <= bound, (k, res[k], bound)
    # every op above is one intercepted GEMM call: fp32 and bf16 through the
    # hipBLAS symbols, fp16 through rocblas_gemm_ex (PyTorch's paths on ROCm)
    calls = [l for l in r.stderr.splitlines() if l.startswith(("[vkblas] hipblas gemm", "[vkblas] rocblas gemm"))]
    assert len(calls) >= len(BOUNDS), r.stderr[-4000:]
    assert "forwarding" not in r.stderr, r.stderr[-4000:]
    assert any("f16->f16" in l for l in calls), calls
    assert any("bf16->bf16" in l for l in calls), calls
    assert any("batch=8" in l for l in calls), calls
    engine = [l for l in r.stderr.splitlines() if l.startswith("[vkblas] gemm ")]
    assert any("path=skinny" in l and "f16->f16" in l and "bf16" not in l for l in engine), engine
    assert any("path=skinny" in l and "bf16->bf16" in l for l in engine), engine


def test_unmodified_script_through_the_runner(tmp_path):
    """python -m vkblas_amd.preload --torch-hipblas -- python script.py: a
    script that never mentions the library has its matmul intercepted."""
    import os
    script = tmp_path / "plain.py"
    script.write_text("import torch\n"
                      "a = torch.rand(300, 200, device='cuda:0'); b = torch.rand(200, 100, device='cuda:0')\n"
                      "c = (a @ b).double().cpu(); r = a.double().cpu() @ b.double().cpu()\n"
                      "print('REL', float((c - r).abs().max() / r.abs().max()))\n")
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, VKBLAS_TRACE="1")
    env["PYTHONPATH"] = os.pathsep.join([repo] + ([env["PYTHONPATH"]] if env.get("PYTHONPATH") else []))
    print("[case] runner --torch-hipblas", flush=True)
    r = subprocess.run([sys.executable, "-m", "vkblas_amd.preload", "--torch-hipblas", "--", sys.executable,
                        str(script)], env=env, cwd=repo, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    rel = float(next(l for l in r.stdout.splitlines() if l.startswith("REL ")).split()[1])
    assert rel <= 1e-5 * 200 ** 0.5
    assert any(l.startswith("[vkblas] hipblas gemm NN f32->f32 m=100 n=300 k=200") for l in r.stderr.splitlines()), \
        r.stderr[-4000:]
