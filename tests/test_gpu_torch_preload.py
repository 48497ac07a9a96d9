"""PyTorch-ROCm with libvkblas_hipblas.so preloaded, the reference's main use
(reference README.md:56-70, test/test_torch.py): torch's matmul, bmm, addmm
and linear must reach this library and give the right answers.  Each case
runs in a child process with the library in LD_PRELOAD; VKBLAS_TRACE=1 makes
the library log every GEMM it takes, so the test can tell an intercepted call
from one that went to the vendor library.  Two backends: PyTorch's default on
gfx950 (hipBLASLt, interposed at hipblasLtMatmul), and its hipBLAS backend
(torch.backends.cuda.preferred_blas_library("cublas")), which calls the
hipBLAS and rocBLAS entry points.
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


# The reference's end-to-end script (test/test_torch.py:10-110), run the way
# its README runs it: LD_PRELOAD naming this library, PyTorch's default
# BLAS backend (hipBLASLt on gfx950), nothing else changed.  Added: linear
# with a bias in fp32 / fp16 / bf16 and addmm with a 1-D bias (hipBLASLt's
# bias epilogue), each checked against PyTorch's CPU result.
CHILD_PLAIN = r"""
import json, torch
torch.manual_seed(42)
dev = "cuda"
out = {}
def diff(got, ref):
    torch.cuda.synchronize()
    got = got.cpu().double(); ref = ref.double()
    return [float((got - ref).abs().max()), float((got - ref).abs().max() / ref.abs().max())]
# test_torch.py:10-25 shapes, fp32 a @ b
for (m, n, k) in [(128, 128, 128), (512, 512, 512), (4096, 4096, 4096), (4096, 1024, 4096), (1024, 4096, 4096),
                  (257, 129, 64), (33, 65, 17), (1, 64, 64), (64, 1, 64), (3, 5, 7)]:
    a = torch.randn(m, k, device=dev); b = torch.randn(k, n, device=dev)
    out[f"mm_{m}x{n}x{k}"] = diff(a @ b, a.cpu() @ b.cpu())
# :28-34 bmm
a = torch.randn(4, 64, 32, device=dev); b = torch.randn(4, 32, 128, device=dev)
out["bmm"] = diff(torch.bmm(a, b), torch.bmm(a.cpu(), b.cpu()))
# :37-43 x @ W.t()
x = torch.randn(128, 256, device=dev); w = torch.randn(512, 256, device=dev)
out["x_wt"] = diff(x @ w.t(), x.cpu() @ w.cpu().t())
# :45-54 non-contiguous x.t() @ w
for (M, K, N) in [(33, 97, 65), (128, 256, 128), (512, 768, 256)]:
    x = torch.randn(K, M, device=dev); w = torch.randn(K, N, device=dev)
    out[f"xt_w_{M}x{K}x{N}"] = diff(x.t() @ w, x.t().cpu() @ w.cpu())
# :56-63 batched transposed A
x = torch.randn(3, 256, 320, device=dev); w = torch.randn(3, 256, 128, device=dev)
out["bmm_xt_w"] = diff(x.transpose(1, 2) @ w, x.transpose(1, 2).cpu() @ w.cpu())
# :65-73 addmm with a 1-D bias, alpha / beta
x = torch.randn(256, 320, device=dev); w = torch.randn(256, 128, device=dev); bias = torch.randn(128, device=dev)
out["addmm_bias_ab"] = diff(torch.addmm(bias, x.t(), w, beta=0.5, alpha=2.5),
                            0.5 * bias.cpu() + 2.5 * (x.t().cpu() @ w.cpu()))
# :75-83 addmm with a matrix C
a = torch.randn(256, 256, device=dev); b = torch.randn(256, 256, device=dev); c = torch.randn(256, 256, device=dev)
out["addmm_c"] = diff(torch.addmm(c, a, b, beta=0.7, alpha=0.5), 0.7 * c.cpu() + 0.5 * (a.cpu() @ b.cpu()))
# :85-91 fp16
a16 = torch.randn(128, 128, device=dev, dtype=torch.float16); b16 = torch.randn(128, 128, device=dev, dtype=torch.float16)
out["mm_f16"] = diff(a16 @ b16, a16.cpu().float() @ b16.cpu().float())
# :93-110 complex128 (forwarded to the vendor library)
for (m, n, k) in [(16, 16, 16), (33, 65, 17), (128, 256, 320), (512, 256, 768)]:
    a = torch.randn(m, k, device=dev, dtype=torch.complex128); b = torch.randn(k, n, device=dev, dtype=torch.complex128)
    torch.cuda.synchronize()
    d = float((a @ b).cpu().sub(a.cpu() @ b.cpu()).abs().max())
    out[f"z64_{m}x{n}x{k}"] = [d, d]
a = torch.randn(3, 64, 32, device=dev, dtype=torch.complex128); b = torch.randn(3, 32, 48, device=dev, dtype=torch.complex128)
d = float(torch.bmm(a, b).cpu().sub(torch.bmm(a.cpu(), b.cpu())).abs().max()); out["z64_bmm"] = [d, d]
x = torch.randn(64, 128, device=dev, dtype=torch.complex128); w = torch.randn(256, 128, device=dev, dtype=torch.complex128)
d = float((x @ w.t()).cpu().sub(x.cpu() @ w.cpu().t()).abs().max()); out["z64_linear"] = [d, d]
# linear with a bias (addmm + hipBLASLt bias epilogue), three dtypes
for name, dt in (("f32", torch.float32), ("f16", torch.float16), ("bf16", torch.bfloat16)):
    x = (torch.randn(64, 512, device=dev) / 16).to(dt); W = torch.randn(384, 512, device=dev).to(dt)
    b = torch.randn(384, device=dev).to(dt)
    out[f"linear_bias_{name}"] = diff(torch.nn.functional.linear(x, W, b),
                                      x.cpu().double() @ W.cpu().double().t() + b.cpu().double())
    xd = torch.randn(4, 512, device=dev).to(dt)      # decode-shaped
    out[f"linear_bias_decode_{name}"] = diff(torch.nn.functional.linear(xd, W, b),
                                             xd.cpu().double() @ W.cpu().double().t() + b.cpu().double())
print("RESULT " + json.dumps(out), flush=True)
"""


def test_plain_ld_preload_reference_script():
    """LD_PRELOAD=libvkblas_hipblas.so python script.py, the reference's
    usage (reference README.md:60-70), with its test_torch.py cases: every fp32 / fp16
    / bf16 product reaches this library through hipblasLtMatmul (bias
    epilogues included) and matches PyTorch's CPU result; complex128 goes to
    the vendor library and is exact to 1e-8 as the reference requires."""
    import os
    import vkblas_amd as vk
    old = os.environ.get("LD_PRELOAD", "")
    # this library first; whatever the environment already preloads stays
    env = dict(os.environ, LD_PRELOAD=":".join([vk.LIB_PATH] + ([old] if old else [])), VKBLAS_TRACE="1")
    print("[case] plain LD_PRELOAD, reference test_torch.py cases", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD_PLAIN], env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    res = json.loads(next(l for l in r.stdout.splitlines() if l.startswith("RESULT "))[len("RESULT "):])
    for key, (absd, rel) in res.items():
        if key.startswith("z64"):
            assert absd < 1e-8, (key, absd)                 # test_torch.py:100
        elif "bf16" in key:
            assert rel <= 8e-3, (key, rel)
        elif "f16" in key:
            assert rel <= 2e-3, (key, rel)
        else:
            assert absd < 0.1, (key, absd)                  # test_torch.py:19
    err = r.stderr.splitlines()
    lt = [l for l in err if l.startswith("[vkblas] hipblaslt matmul")]
    assert len(lt) >= 20, r.stderr[-4000:]
    assert sum(" bias" in l for l in lt) >= 6, lt           # six linear(x, W, b) calls
    assert any("f16->f16" in l and " bias" in l for l in lt), lt
    assert any("bf16->bf16" in l and " bias" in l for l in lt), lt
    assert any("f32->f32" in l and "m=4096 n=4096 k=4096" in l for l in lt), lt
    assert not any("forwarding" in l for l in err), r.stderr[-4000:]
    # the kernels ran in the same process, on PyTorch's HIP runtime
    assert any(l.startswith("[vkblas] gemm ") and "path=skinny" in l for l in err), r.stderr[-4000:]


# Seeded random PyTorch products under plain LD_PRELOAD: matmul of 2-D
# tensors (contiguous or transposed views), bmm and batched matmul (right
# operand contiguous: PyTorch's own bf16 batched path has faulted on a
# transposed right operand on these boxes), linear with and without a bias,
# addmm with alpha / beta and a matrix or 1-D bias, decode-shaped linear;
# fp32, fp16 and bf16.  Each result is checked against PyTorch's CPU result
# in float64 of the same inputs (normwise: fp32 1e-5 sqrt(K), fp16 2e-3,
# bf16 8e-3), and no call may be forwarded to the vendor library.
CHILD_RANDOM = r"""
import json, math, torch
g = torch.Generator().manual_seed(2026)
dev = "cuda"
out = []
DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
def ri(lo, hi):
    return int(torch.randint(lo, hi + 1, (1,), generator=g))
def rnd(*shape, dt, scale=1.0):
    return (torch.randn(*shape, generator=g) * scale).to(DT[dt])
def rel(got, ref):
    torch.cuda.synchronize()
    got = got.cpu().double(); ref = ref.double()
    den = float(ref.abs().max())
    return float((got - ref).abs().max()) / (den if den > 0 else 1.0)
for i in range(120):
    dt = ["f32", "f16", "bf16"][i % 3]
    kind = ["mm", "mm_t", "bmm", "linear", "linear_bias", "addmm", "decode"][ri(0, 6)]
    big = ri(0, 9) == 0
    M, N, K = (ri(1, 3000), ri(1, 3000), ri(1, 2048)) if big else (ri(1, 400), ri(1, 400), ri(1, 600))
    if ri(0, 1):
        M, N, K = -(-M // 8) * 8, -(-N // 8) * 8, -(-K // 8) * 8
    s = 1.0 / math.sqrt(K)
    if kind == "mm":
        a, b = rnd(M, K, dt=dt), rnd(K, N, dt=dt, scale=s)
        got, ref = a.to(dev) @ b.to(dev), a.double() @ b.double()
    elif kind == "mm_t":     # transposed views on either side
        a, b = rnd(K, M, dt=dt), rnd(N, K, dt=dt, scale=s)
        got, ref = a.to(dev).t() @ b.to(dev).t(), a.double().t() @ b.double().t()
    elif kind == "bmm":
        B = ri(2, 4)
        a, b = rnd(B, M if not big else M // 8 + 1, K, dt=dt), rnd(B, K, N if not big else N // 8 + 1, dt=dt, scale=s)
        got, ref = torch.bmm(a.to(dev), b.to(dev).contiguous()), torch.bmm(a.double(), b.double())
    elif kind in ("linear", "linear_bias"):
        x, w = rnd(M, K, dt=dt), rnd(N, K, dt=dt, scale=s)
        bias = rnd(N, dt=dt) if kind == "linear_bias" else None
        got = torch.nn.functional.linear(x.to(dev), w.to(dev), None if bias is None else bias.to(dev))
        ref = x.double() @ w.double().t() + (0 if bias is None else bias.double())
    elif kind == "addmm":
        a, b = rnd(M, K, dt=dt), rnd(K, N, dt=dt, scale=s)
        c = rnd(N, dt=dt) if ri(0, 1) else rnd(M, N, dt=dt)
        al, be = round(float(torch.rand(1, generator=g)) * 3 - 1.5, 3), round(float(torch.rand(1, generator=g)) * 2 - 1, 3)
        got = torch.addmm(c.to(dev), a.to(dev), b.to(dev), beta=be, alpha=al)
        ref = be * c.double() + al * (a.double() @ b.double())
    else:                    # decode: a few tokens against a large weight
        T = ri(1, 16)
        O, K2 = -(-ri(256, 8192) // 8) * 8, -(-ri(256, 4096) // 8) * 8
        x, w = rnd(T, K2, dt=dt), rnd(O, K2, dt=dt, scale=1.0 / math.sqrt(K2))
        got, ref = torch.nn.functional.linear(x.to(dev), w.to(dev)), x.double() @ w.double().t()
        K = K2
    out.append([i, kind, dt, K, rel(got, ref)])
print("RESULT " + json.dumps(out), flush=True)
"""


def test_plain_ld_preload_random_products():
    import os
    import vkblas_amd as vk
    old = os.environ.get("LD_PRELOAD", "")
    env = dict(os.environ, LD_PRELOAD=":".join([vk.LIB_PATH] + ([old] if old else [])), VKBLAS_TRACE="1")
    print("[case] plain LD_PRELOAD, 120 seeded random products", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD_RANDOM], env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    res = json.loads(next(l for l in r.stdout.splitlines() if l.startswith("RESULT "))[len("RESULT "):])
    assert len(res) == 120
    for i, kind, dt, K, err in res:
        bound = 8e-3 if dt == "bf16" else 2e-3 if dt == "f16" else 1e-5 * K ** 0.5
        assert err <= bound, (i, kind, dt, K, err)
    err_lines = r.stderr.splitlines()
    assert not any("forwarding" in l for l in err_lines), [l for l in err_lines if "forwarding" in l][:5]
    assert sum(l.startswith("[vkblas] gemm ") for l in err_lines) >= 120, r.stderr[-2000:]


# torch.cuda.graph under plain LD_PRELOAD: a step of products whose plans
# need no partials (a 256-token linear on 64x64 tiles, 8-token and 1-token
# decode linears, a 512^3 matmul) captured through the interposed
# hipblasLtMatmul, replayed three times with eager steps between the
# replays; every replay equals the eager step bit for bit.
CHILD_GRAPH = r"""
import json, torch
dev = "cuda"
torch.manual_seed(3)
W1 = (torch.randn(1024, 1024, device=dev) * 0.03).half()
W2 = (torch.randn(4096, 4096, device=dev) * 0.015).half()
x1 = torch.randn(256, 1024, device=dev).half()
x2 = torch.randn(8, 4096, device=dev).half()
x3 = torch.randn(1, 4096, device=dev).half()
a = torch.randn(512, 512, device=dev).half(); b = (torch.randn(512, 512, device=dev) * 0.05).half()
def step():
    return [x1 @ W1.t(), x2 @ W2.t(), x3 @ W2.t(), a @ b]
eager = [t.clone() for t in step()]
torch.cuda.synchronize()
s = torch.cuda.Stream(); s.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(s):
    for _ in range(2):
        step()
torch.cuda.current_stream().wait_stream(s)
torch.cuda.synchronize()
print("CAPTURE", flush=True)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    outs = step()
res = []
for rep in range(3):
    for o in outs:
        o.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    res.append([bool(torch.equal(o, e)) for o, e in zip(outs, eager)])
    again = step()
    torch.cuda.synchronize()
    res.append([bool(torch.equal(o, e)) for o, e in zip(again, eager)])
print("RESULT " + json.dumps(res), flush=True)
"""


def test_plain_ld_preload_graph_capture_without_partials():
    import os
    import vkblas_amd as vk
    # the step's calls, in the engine's row-major form, need no partials
    for M, N, K in ((256, 1024, 1024), (8, 4096, 4096), (1, 4096, 4096)):
        pl = vk.plan(vk.DT_F16, vk.DT_F16, 0, 1, M, N, K, K, K, N)
        assert pl.split == 1 and pl.path not in (vk.PATH_SPLITK, vk.PATH_TAIL), (M, N, K, pl.path, pl.split)
    pl = vk.plan(vk.DT_F16, vk.DT_F16, 0, 0, 512, 512, 512, 512, 512, 512)
    assert pl.split == 1 and pl.path not in (vk.PATH_SPLITK, vk.PATH_TAIL)
    old = os.environ.get("LD_PRELOAD", "")
    env = dict(os.environ, LD_PRELOAD=":".join([vk.LIB_PATH] + ([old] if old else [])), VKBLAS_TRACE="1")
    print("[case] plain LD_PRELOAD, torch.cuda.graph of products without partials", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD_GRAPH], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
    res = json.loads(next(l for l in r.stdout.splitlines() if l.startswith("RESULT "))[len("RESULT "):])
    assert res and all(all(x) for x in res), res
    err = r.stderr.splitlines()
    assert not any("forwarding" in l for l in err), [l for l in err if "forwarding" in l][:5]
    assert not any("declined" in l for l in err), [l for l in err if "declined" in l][:5]
    assert sum(l.startswith("[vkblas] hipblaslt matmul") for l in err) >= 4 * 4, r.stderr[-2000:]
