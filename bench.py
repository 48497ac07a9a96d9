#!/usr/bin/env python3
"""Benchmark of the MI355X-native vkblas GEMM hot path (one GPU).

Headline: fp32 GEMM M=N=K=4096, column-major,
ld=4096, alpha=1, beta=0, all four transpose variants.  One step = the four
variants NN, NT, TN, TT back to back through the library's hipblasSgemm
(C ABI, a hipBLAS handle on the timed stream).  value = total
algorithmic FLOPs (2*M*N*K per GEMM) / wall time of the K timed steps.

The same run also reports the other BASELINE targets (fp16 4096^3 GEMM vs the
fp16 MFMA peak, 8192x8192 fp16 decode matvec vs HBM peak, with three weight
copies rotated so the 256 MB Infinity Cache cannot serve them), a roofline
object for the dominant kernel and the CPU comparator.

  python bench.py [--gpus 1] [--steps K] [--warmup W]
                  [--only fp32|fp16|bf16|matvec|matvec_ns|bf16mv|f32mv|splitk|batched|shapes|ceiling|vendor]
"""
import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

PEAK_FP32_TFLOPS = 157.3     # MI355X dense fp32 matrix
PEAK_FP16_TFLOPS = 2516.6    # MI355X dense fp16 MFMA (no sparsity)
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E

# HBM bytes per launch of the fp32 4096^3 256x256 GEMM kernel: rocprofv3
# FETCH_SIZE and WRITE_SIZE passes over this benchmark (KiB per dispatch,
# averaged over the four variants), scaled by what the same counters read
# for a 256 MiB device copy (FETCH x2.00, WRITE x1.00).  Summary:
# profiles/hbm_traffic_bench_legs.txt.
TRAFFIC_F32_4096_BYTES = int((2.00 * 196933.1 + 1.00 * 65558.2) * 1024)

METRIC = "TFLOPS 4096³ fp32/fp16 GEMM (% MFMA peak); fp16 matvec GB/s (% HBM peak)"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


WARM_MS = 20.0


def warm(torch, fn, ms=WARM_MS):
    """Untimed launches fn(i), ten at a time, until `ms` of wall time have
    passed: from a cold start (fresh buffers, the GPU idle during host work)
    the first milliseconds of a leg ran up to 15 % slower than the steady
    state (fp16 4096^3: 109-116 against 100 us), which three warmup launches
    did not cover."""
    i = 0
    t0 = time.perf_counter()
    while True:
        for _ in range(10):
            fn(i)
            i += 1
        torch.cuda.synchronize()
        if (time.perf_counter() - t0) * 1e3 >= ms:
            return i


def batch_ms(torch, stream, fn, launches, batches=5):
    """Median over `batches` of the average launch duration of `launches`
    back-to-back calls fn(i) between one pair of HIP events on `stream` (a
    per-launch event pair adds its own gap to a launch of a few tens of us)."""
    avgs, i = [], 0
    for _ in range(batches):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        for _ in range(launches):
            fn(i)
            i += 1
        e.record(stream)
        torch.cuda.synchronize()
        avgs.append(s.elapsed_time(e) / launches)
    avgs.sort()
    return avgs[len(avgs) // 2]


def fp32_headline(torch, vk, stream, steps, warmup):
    """the four hipBLAS transpose variants at 4096^3."""
    n = 4096
    g = torch.Generator(device="cuda:0").manual_seed(2024)
    A = torch.rand(n * n, device="cuda:0", generator=g) * 2 - 1
    B = torch.rand(n * n, device="cuda:0", generator=g) * 2 - 1
    C = torch.empty(n * n, device="cuda:0")
    sp = stream.cuda_stream
    # through the hipBLAS entry point the north star names: hipblasSgemm on a
    # handle whose stream is the timed stream
    import ctypes
    from vkblas_amd import hipblas_abi as hb
    abi = vk.hipblas()
    handle = abi.create()
    if abi.hipblasSetStream(handle, sp) != hb.HIPBLAS_STATUS_SUCCESS:
        raise RuntimeError("hipblasSetStream failed")
    one, zero = ctypes.c_float(1.0), ctypes.c_float(0.0)
    ops = (hb.HIPBLAS_OP_N, hb.HIPBLAS_OP_T)
    pa, pb, pc = A.data_ptr(), B.data_ptr(), C.data_ptr()

    def call(ta, tb):
        st = abi.hipblasSgemm(handle, ops[ta], ops[tb], n, n, n, ctypes.byref(one), pa, n, pb, n, ctypes.byref(zero),
                              pc, n)
        if st != hb.HIPBLAS_STATUS_SUCCESS:
            raise RuntimeError(f"hipblasSgemm failed: {st}")

    variants = [(0, 0), (0, 1), (1, 0), (1, 1)]
    for _ in range(warmup):
        for v in variants:
            call(*v)
    torch.cuda.synchronize()
    # One HIP event pair around the whole timed region, on the launch stream:
    # an event recorded between two launches of this kernel delays the next
    # launch by about 10 us (kernel trace: 0 us between back-to-back launches,
    # 10.2 us median with an event pair around every launch).
    s_ev, e_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    s_ev.record(stream)
    for _ in range(steps):
        for v in variants:
            call(*v)
    e_ev.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    launches = 4 * steps
    avg_ms = s_ev.elapsed_time(e_ev) / launches
    path = vk.PATH_NAMES[vk.last_path()]
    flops = 2.0 * n ** 3
    # per variant, after the timed region: back-to-back launches of one
    # variant between one event pair (batch_ms)
    by_variant = {}
    for ta, tb in variants:
        ms = batch_ms(torch, stream, lambda i, ta=ta, tb=tb: call(ta, tb), max(steps, 10), batches=3)
        by_variant["NT"[ta] + "NT"[tb]] = round(flops / (ms * 1e-3) / 1e12, 2)
    abi.hipblasDestroy(handle)
    return {"wall_s": wall, "flops": flops * launches, "avg_launch_ms": avg_ms, "path": path,
            "tflops_by_variant": by_variant, "launches": launches}


def fp16_gemm(torch, vk, stream, steps, n=4096, bf16=False, f32_out=False):
    """configs[2] sample: fp16 GemmEx 16F x 16F -> 16F, NN and TN (bf16: the
    same with 16BF data and result); with f32_out also 16F x 16F -> 32F."""
    dt = torch.bfloat16 if bf16 else torch.float16
    vdt = vk.DT_BF16 if bf16 else vk.DT_F16
    g = torch.Generator(device="cuda:0").manual_seed(7)
    A = (torch.randn(n * n, device="cuda:0", generator=g) / math.sqrt(n)).to(dt)
    B = (torch.randn(n * n, device="cuda:0", generator=g) / math.sqrt(n)).to(dt)
    C = torch.empty(n * n, device="cuda:0", dtype=torch.float32 if f32_out else dt)
    sp = stream.cuda_stream
    out = {}
    cases = [("NN", 0, vdt), ("TN", 1, vdt)]
    if f32_out:
        cases += [("NN_f32out", 0, vk.DT_F32), ("TN_f32out", 1, vk.DT_F32)]
    for name, ta, cdt in cases:
        def call():
            vk.gemm_async(vdt, cdt, vk.OP_N, ta, n, n, n, 1.0, B.data_ptr(), n, A.data_ptr(), n, 0.0,
                          C.data_ptr(), n, stream=sp)
        warm(torch, lambda i: call())
        med = batch_ms(torch, stream, lambda i: call(), max(steps, 20))
        out[name] = {"ms": round(med, 4), "tflops": round(2.0 * n ** 3 / (med * 1e-3) / 1e12, 1),
                     "path": vk.PATH_NAMES[vk.last_path()]}
        out[name]["frac_of_peak"] = round(out[name]["tflops"] / PEAK_FP16_TFLOPS, 4)
    return out


def shapes(torch, vk, stream, steps):
    """GEMMs off the BASELINE sizes, hipBLAS NN and TN (column-major m x n x
    k) through the planner: fp32 squares on 128x128 tiles (2048^3 one wave;
    3072^3 and 5120^3 with a split tail after whole waves; 6144^3), fp16
    3072^3 (144 tiles of 256x256) and 6144^3 (split tail), and ragged shapes
    on the pipelined kernel's shifted edge tiles (m = 4000, a 2047-token
    fp16 projection)."""
    out = {}
    sp = stream.cuda_stream
    cases = [("f32", 2048, 2048, 2048), ("f32", 3072, 3072, 3072), ("f32", 5120, 5120, 5120),
             ("f32", 6144, 6144, 6144), ("f16", 3072, 3072, 3072), ("f16", 6144, 6144, 6144),
             ("f32", 4000, 4000, 4096), ("f16", 4000, 4000, 4096), ("f16", 14336, 2047, 4096)]
    for dtn, m, n, k in cases:
        g = torch.Generator(device="cuda:0").manual_seed(11)
        A = torch.rand(m * k, device="cuda:0", generator=g) * 2 - 1
        B = torch.rand(k * n, device="cuda:0", generator=g) * 2 - 1
        if dtn == "f16":
            A, B = A.half(), B.half()
        C = torch.empty(m * n, device="cuda:0", dtype=A.dtype)
        vdt = vk.DT_F16 if dtn == "f16" else vk.DT_F32
        peak = PEAK_FP16_TFLOPS if dtn == "f16" else PEAK_FP32_TFLOPS
        for name, ta in (("NN", 0), ("TN", 1)):
            # column-major C (m x n) = op(A) B: the engine computes the
            # row-major n x m product with A and B swapped
            def call():
                vk.gemm_async(vdt, vdt, vk.OP_N, ta, n, m, k, 1.0, B.data_ptr(), k, A.data_ptr(), k if ta else m,
                              0.0, C.data_ptr(), m, stream=sp)
            warm(torch, lambda i: call())
            med = batch_ms(torch, stream, lambda i: call(), max(steps, 10))
            tf = 2.0 * m * n * k / (med * 1e-3) / 1e12
            key = f"{dtn}_{m}" if m == n == k else f"{dtn}_{m}x{n}x{k}"
            out[f"{key}_{name}"] = {"ms": round(med, 4), "tflops": round(tf, 1),
                                    "path": vk.PATH_NAMES[vk.last_path()], "frac_of_peak": round(tf / peak, 4)}
        del A, B, C
    return out


def matvec(torch, vk, stream, steps, K=8192, O=8192, ntoks=(1, 4, 8, 16), bf16=False, kxo=False):
    """decode GemmEx(T, N, m=O, n=ntok, k=K), W K-contiguous;
    three weight copies (3 x 128 MiB > 256 MB MALL) rotated per launch
    (bf16: the same with 16BF data; kxo: the weight stored K x O instead,
    GemmEx(N, N), PyTorch's x @ w)."""
    dt = torch.bfloat16 if bf16 else torch.float16
    vdt = vk.DT_BF16 if bf16 else vk.DT_F16
    g = torch.Generator(device="cuda:0").manual_seed(11)
    Ws = [(torch.randn(O * K, device="cuda:0", generator=g) * 0.02).to(dt) for _ in range(3)]
    X = torch.randn(max(ntoks) * K, device="cuda:0", generator=g).to(dt)
    Y = torch.empty(max(ntoks) * O, device="cuda:0", dtype=dt)
    sp = stream.cuda_stream
    out = {}
    for nt in ntoks:
        def call(i):
            vk.gemm_async(vdt, vdt, vk.OP_N, vk.OP_N if kxo else vk.OP_T, nt, O, K, 1.0, X.data_ptr(), K,
                          Ws[i % 3].data_ptr(), O if kxo else K, 0.0, Y.data_ptr(), O, stream=sp)
        warm(torch, call)
        med = batch_ms(torch, stream, call, 3 * max(steps, 10))
        nbytes = 2 * O * K + 2 * K * nt + 2 * O * nt
        gbs = nbytes / (med * 1e-3) / 1e9
        out[f"n{nt}"] = {"us": round(med * 1e3, 2), "GBps": round(gbs, 1), "frac_of_hbm": round(gbs / PEAK_HBM_GBS, 4),
                         "path": vk.PATH_NAMES[vk.last_path()]}
    return out


def matvec_f32(torch, vk, stream, steps, K=8192, O=8192, ntoks=(1, 4, 8, 16)):
    """fp32 decode (the reference's fp32 matvec, src/vkblas.c:2100-2143):
    Y[ntok][O] = X[ntok][K] . W with W
    stored O x K (engine op_b = T, hipBLAS TN) and K x O (op_b = N, hipBLAS
    NN); three weight copies (3 x 256 MiB > 256 MB MALL) rotated per launch."""
    g = torch.Generator(device="cuda:0").manual_seed(17)
    Ws = [torch.randn(O * K, device="cuda:0", generator=g) * 0.02 for _ in range(3)]
    X = torch.randn(max(ntoks) * K, device="cuda:0", generator=g)
    Y = torch.empty(max(ntoks) * O, device="cuda:0")
    sp = stream.cuda_stream
    out = {}
    for name, ob in (("OxK", vk.OP_T), ("KxO", vk.OP_N)):
        ldw = K if ob == vk.OP_T else O
        for nt in ntoks:
            def call(i):
                vk.gemm_async(vk.DT_F32, vk.DT_F32, vk.OP_N, ob, nt, O, K, 1.0, X.data_ptr(), K,
                              Ws[i % 3].data_ptr(), ldw, 0.0, Y.data_ptr(), O, stream=sp)
            warm(torch, call)
            med = batch_ms(torch, stream, call, 3 * max(steps, 10))
            nbytes = 4 * O * K + 4 * K * nt + 4 * O * nt
            gbs = nbytes / (med * 1e-3) / 1e9
            out[f"{name}_n{nt}"] = {"us": round(med * 1e3, 2), "GBps": round(gbs, 1),
                                    "frac_of_hbm": round(gbs / PEAK_HBM_GBS, 4),
                                    "path": vk.PATH_NAMES[vk.last_path()]}
    return out


def mfma_ceiling(torch, vk, stream, steps):
    """The v_mfma_f32_16x16x32 rate the chip sustains with no memory traffic
    (vkblas_mfma_probe: the GEMM inner loop's MFMA pattern without its loads),
    on operands drawn as the 16-bit legs' data (N(0,1)/sqrt(4096)) and on
    zeros.  Under the power limit this rate depends on the data; it is the
    ceiling the 16-bit GEMM legs' frac_of_peak is held to."""
    from vkblas_amd import bench_probe as probe
    sp = stream.cuda_stream
    blocks, iters = 256, 320                     # 172 GFLOP a launch, as long as a 4096^3 GEMM
    flops = blocks * 4 * iters * 32 * 16 * 16 * 32 * 2
    out = torch.empty(blocks * 256, device="cuda:0")
    g = torch.Generator(device="cuda:0").manual_seed(13)
    res = {}
    for name, bf16 in (("fp16", False), ("bf16", True)):
        dt = torch.bfloat16 if bf16 else torch.float16
        for data in ("normal", "zeros"):
            ops = torch.randn(12 * 64 * 8, device="cuda:0", generator=g) / 64.0
            ops = (ops if data == "normal" else torch.zeros_like(ops)).to(dt)

            def call(i):
                probe.mfma_probe(bf16, ops.data_ptr(), out.data_ptr(), blocks, iters, stream=sp)
            warm(torch, call)
            med = batch_ms(torch, stream, call, max(steps, 20))
            tf = flops / (med * 1e-3) / 1e12
            res[f"{name}_{data}"] = {"tflops": round(tf, 1), "frac_of_peak": round(tf / PEAK_FP16_TFLOPS, 4)}
    return res


def copy_ceiling(torch, vk, stream, steps):
    """The rate at which a CU copies GEMM operand tiles from L2 into LDS
    (vkblas_copy_probe: the 256x256 fp16 tile's buffer -> LDS copies at 4096^3
    with no compute), with one step of copies in flight (waited for at each
    step's end, as the two-stage GEMM kernel) or two, rows of 128 bytes (the
    GEMM kernel's) or 64, on 256 workgroups (one per CU) or fewer.  The copies
    of a 4096^3 (2048^3) 16-bit GEMM on 256x256 (128x128) tiles are 4 MiB (1
    MiB) per CU: this rate bounds how fast they can be done."""
    from vkblas_amd import bench_probe as probe
    n = 4096
    g = torch.Generator(device="cuda:0").manual_seed(19)
    A = (torch.randn(n * n, device="cuda:0", generator=g) / 64.0).half()
    B = (torch.randn(n * n, device="cuda:0", generator=g) / 64.0).half()
    out = torch.empty(256, device="cuda:0", dtype=torch.int32)
    sp = stream.cuda_stream
    res = {}
    for d, rb, blocks in ((1, 128, 256), (2, 128, 256), (2, 64, 256), (2, 128, 64), (2, 128, 8)):
        def call(i):
            probe.copy_probe(A.data_ptr(), B.data_ptr(), n, blocks, d, rb, out.data_ptr(), stream=sp)
        warm(torch, call)
        med = batch_ms(torch, stream, call, max(steps, 20))
        nbytes = blocks * n * 2 * 256 * 2          # every K step of A and B rows of each tile
        res[f"inflight{d}_row{rb}_wg{blocks}"] = {"us": round(med * 1e3, 2),
                                                  "GBps_per_cu": round(nbytes / blocks / (med * 1e-3) / 1e9, 1),
                                                  "TBps": round(nbytes / (med * 1e-3) / 1e12, 2)}
    return res


def cpu_baseline(budget_s=12.0):
    """The reference's CPU GEMM (test/test_gemm.c:32-58, restated in
    oracle/ref_gemm.c) on the headline workload, NN, parallel over output
    columns on every host core; row-sampled as test_gemm.c does and scaled to
    the full 4096 rows."""
    import numpy as np
    import oracle
    n = 4096
    threads = os.cpu_count() or 1
    try:
        threads = len(os.sched_getaffinity(0))
    except Exception:
        pass
    r = np.random.default_rng(5)
    A = r.uniform(-1, 1, n * n).astype(np.float32)
    B = r.uniform(-1, 1, n * n).astype(np.float32)
    C = np.zeros(n * n, np.float32)
    rows = 12
    t0 = time.perf_counter()
    oracle.ref_gemm_cm(0, 0, n, n, n, 1.0, A, n, B, n, 0.0, C, n, rows, threads=threads)
    t = time.perf_counter() - t0
    # grow the sample to fill about budget_s of CPU time
    if t < budget_s / 4:
        rows = int(min(n, max(12, rows * (budget_s / max(t, 1e-3)))))
        t0 = time.perf_counter()
        oracle.ref_gemm_cm(0, 0, n, n, n, 1.0, A, n, B, n, 0.0, C, n, rows, threads=threads)
        t = time.perf_counter() - t0
    gflops = 2.0 * rows * n * n / t / 1e9
    return {"value": round(gflops / 1e3, 5), "unit": "TFLOPS", "cores": threads, "kind": "port",
            "sample": f"fp32 NN 4096^3, {rows} of 4096 rows (test_gemm.c row sampling), {t:.1f} s, "
                      f"double accumulation, OpenMP over columns; {gflops:.2f} GFLOP/s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=["fp32", "fp16", "bf16", "matvec", "matvec_ns", "bf16mv", "f32mv", "splitk", "batched",
                                       "shapes", "calibrate", "ceiling", "vendor"],
                    default=None)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--splits", default="4,16,64,0",
                    help="--only splitk: the splits to time (0: the planner's choice)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the GEMM hot path has no multi-GPU path in this build "
              "(each GPU would run its own GEMMs on its own stream). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import vkblas_amd as vk
    vk.load()
    stream = torch.cuda.current_stream()

    if args.only == "fp16":
        print(json.dumps({n: fp16_gemm(torch, vk, stream, args.steps, n=n) for n in (2048, 4096, 8192)}))
        return
    if args.only == "bf16":
        print(json.dumps(fp16_gemm(torch, vk, stream, args.steps, bf16=True)))
        return
    if args.only == "matvec":
        print(json.dumps({"n1-16": matvec(torch, vk, stream, args.steps),
                          "n24-64": matvec(torch, vk, stream, args.steps, ntoks=(24, 32, 64)),
                          "KxO_n1-16": matvec(torch, vk, stream, args.steps, kxo=True)}))
        return
    if args.only == "matvec_ns":
        print(json.dumps({"4096x14336": matvec(torch, vk, stream, args.steps, K=4096, O=14336, ntoks=(1, 4, 8, 12, 16)),
                          "14336x4096": matvec(torch, vk, stream, args.steps, K=14336, O=4096, ntoks=(1, 4, 8, 12, 16))}))
        return
    if args.only == "bf16mv":
        print(json.dumps(matvec(torch, vk, stream, args.steps, bf16=True)))
        return
    if args.only == "f32mv":
        print(json.dumps({"8192x8192": matvec_f32(torch, vk, stream, args.steps),
                          "4096x14336": matvec_f32(torch, vk, stream, args.steps, K=4096, O=14336),
                          "14336x4096": matvec_f32(torch, vk, stream, args.steps, K=14336, O=4096)}))
        return
    if args.only == "splitk":
        splits = tuple(int(x) for x in args.splits.split(","))
        print(json.dumps(splitk(torch, vk, stream, args.steps, splits=splits)))
        return
    if args.only == "batched":
        print(json.dumps(batched(torch, vk, stream, args.steps)))
        return
    if args.only == "shapes":
        print(json.dumps(shapes(torch, vk, stream, args.steps)))
        return
    if args.only == "vendor":
        print(json.dumps(vendor(torch, vk, stream, args.steps)))
        return
    if args.only == "ceiling":
        print(json.dumps({"mfma": mfma_ceiling(torch, vk, stream, args.steps),
                          "copy": copy_ceiling(torch, vk, stream, args.steps)}))
        return
    if args.only == "calibrate":
        print(json.dumps(calibrate(torch, stream)))
        return
    if args.only == "fp32":
        h = fp32_headline(torch, vk, stream, args.steps, args.warmup)
        print(json.dumps(h))
        return

    log("[bench] fp32 4096^3 x 4 variants")
    h = fp32_headline(torch, vk, stream, args.steps, args.warmup)
    value = h["flops"] / h["wall_s"] / 1e12
    achieved = 2.0 * 4096 ** 3 / (h["avg_launch_ms"] * 1e-3) / 1e12
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["wall_s"] * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: U[-1,1) fp32 from a seeded generator, inputs resident in HBM",
        "config": {"workload": "fp32 GEMM M=N=K=4096, column-major ld=4096, alpha=1, beta=0, "
                               "hipBLAS NN+NT+TN+TT per step (BASELINE configs[1])",
                   "M": 4096, "N": 4096, "K": 4096, "variants": ["NN", "NT", "TN", "TT"],
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": TRAFFIC_F32_4096_BYTES,
                     "traffic_note": "HBM bytes per launch from rocprofv3 FETCH_SIZE/WRITE_SIZE (copy-calibrated); "
                                     "algorithmic A+B+C = 201326592 B",
                     "kernel": f"gemm_pipe_kernel<float,float,*,*> ({h['path']})",
                     "algorithmic": "2*4096^3 FLOP per launch"},
        "tflops_by_variant": h["tflops_by_variant"],
    }
    log("[bench] fp16 4096^3")
    line["fp16_gemm_4096"] = fp16_gemm(torch, vk, stream, args.steps, f32_out=True)
    log("[bench] MFMA rate without memory traffic (power-limited ceiling of the 16-bit legs)")
    line["mfma_ceiling"] = mfma_ceiling(torch, vk, stream, args.steps)
    log("[bench] L2 -> LDS copy rate without compute (the 16-bit GEMMs' copy ceiling)")
    line["copy_ceiling"] = copy_ceiling(torch, vk, stream, args.steps)
    log("[bench] fp16 matvec 8192x8192")
    line["fp16_matvec_8192"] = matvec(torch, vk, stream, args.steps)
    log("[bench] bf16 4096^3")
    line["bf16_gemm_4096"] = fp16_gemm(torch, vk, stream, args.steps, bf16=True)
    log("[bench] bf16 matvec 8192x8192")
    line["bf16_matvec_8192"] = matvec(torch, vk, stream, args.steps, ntoks=(1, 8), bf16=True)
    log("[bench] fp16 2048^3 and 8192^3")
    line["fp16_gemm_2048"] = fp16_gemm(torch, vk, stream, args.steps, n=2048, f32_out=True)
    line["fp16_gemm_8192"] = fp16_gemm(torch, vk, stream, args.steps, n=8192, f32_out=True)
    log("[bench] decode 4096x14336 / 14336x4096")
    line["fp16_matvec_4096x14336"] = matvec(torch, vk, stream, args.steps, K=4096, O=14336, ntoks=(1, 4, 8, 16))
    line["fp16_matvec_14336x4096"] = matvec(torch, vk, stream, args.steps, K=14336, O=4096, ntoks=(1, 4, 8, 16))
    log("[bench] decode 8192x8192, 24-64 tokens")
    line["fp16_decode_8192_wide"] = matvec(torch, vk, stream, args.steps, ntoks=(24, 32, 64))
    log("[bench] fp16 matvec 8192x8192, weight stored K x O")
    line["fp16_matvec_8192_KxO"] = matvec(torch, vk, stream, args.steps, ntoks=(1, 8, 16, 32), kxo=True)
    log("[bench] fp32 matvec 8192x8192, both weight layouts")
    line["fp32_matvec_8192"] = matvec_f32(torch, vk, stream, args.steps)
    line["fp32_decode_8192_wide"] = matvec_f32(torch, vk, stream, args.steps, ntoks=(32, 64))
    log("[bench] split-K and strided-batched")
    line["splitk_256x256"] = splitk(torch, vk, stream, args.steps)
    line["batched_fp32_64x512"] = batched(torch, vk, stream, args.steps)
    log("[bench] square GEMMs off the BASELINE sizes")
    line["more_shapes"] = shapes(torch, vk, stream, args.steps)
    if not args.no_cpu:
        # last, so the GPU legs run back to back without an idle gap between them
        log("[bench] cpu baseline")
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


def calibrate(torch, stream, mib=256, reps=5):
    """A plain device copy of known size (torch's copy kernel), so that
    rocprofv3's FETCH_SIZE / WRITE_SIZE can be scaled to bytes."""
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    ts = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record(stream)
        dst.copy_(src)
        e.record(stream)
        torch.cuda.synchronize()
        ts.append(s.elapsed_time(e))
    return {"copy_bytes_read": n, "copy_bytes_written": n, "ms": sorted(ts)[len(ts) // 2]}


def splitk(torch, vk, stream, steps, splits=(4, 16, 64, 0)):
    """M=N=256 tall-K split-K, fp32 and fp16, split {4,16,64} and the planner's choice (0)."""
    sp = stream.cuda_stream
    out = {}
    for K in (65536, 262144):
        for dt in ("f32", "f16"):
            A = torch.rand(256 * K, device="cuda:0") * 2 - 1
            B = torch.rand(K * 256, device="cuda:0") * 2 - 1
            if dt == "f16":
                A, B = A.half(), B.half()
            C = torch.empty(256 * 256, device="cuda:0")
            for split in splits:
                def call():
                    vk.gemm_async(vk.DT_F16 if dt == "f16" else vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, K, 1.0,
                                  A.data_ptr(), K, B.data_ptr(), 256, 0.0, C.data_ptr(), 256, split_k=split,
                                  stream=sp)
                warm(torch, lambda i: call())
                med = batch_ms(torch, stream, lambda i: call(), max(steps, 10))
                tf = 2.0 * 256 * 256 * K / (med * 1e-3) / 1e12
                gbs = (A.numel() + B.numel()) * A.element_size() / (med * 1e-3) / 1e9
                key = f"K{K}_{dt}_s{split}" if split else f"K{K}_{dt}_auto"
                out[key] = {"ms": round(med, 4), "tflops": round(tf, 2), "GBps": round(gbs, 1),
                            "frac_of_mfma": round(tf / (PEAK_FP16_TFLOPS if dt == "f16" else PEAK_FP32_TFLOPS), 4),
                            "frac_of_hbm": round(gbs / PEAK_HBM_GBS, 4)}
                if not split:
                    pl = vk.plan(vk.DT_F16 if dt == "f16" else vk.DT_F32, vk.DT_F32, 0, 0, 256, 256, K, K, 256, 256)
                    out[key]["split"] = pl.split
                    out[key]["tile"] = {0: 64, 1: 128, 2: 256, 3: 32, 4: 64}[pl.tile]
            del A, B
    return out


def vendor(torch, vk, stream, steps):
    """The same workloads through PyTorch's own GEMM backend (hipBLASLt on
    gfx950), timed like the vkblas legs: fp32 / fp16 / bf16 4096^3 (row-major
    a @ b and a @ b.t(), i.e. hipBLAS NN and TN), the `shapes` leg's GEMMs
    (a @ b) and 8192x8192 fp16 decode x @ w.t() and x @ w with three weight
    copies rotated.  Not part of the default run: the library-against-vendor
    comparison is run from here (plain, and with libvkblas_hipblas.so under
    LD_PRELOAD)."""
    n = 4096
    g = torch.Generator(device="cuda:0").manual_seed(7)
    out = {}
    for name, dt in (("fp32", torch.float32), ("fp16", torch.float16), ("bf16", torch.bfloat16)):
        a = (torch.randn(n, n, device="cuda:0", generator=g) / math.sqrt(n)).to(dt)
        b = (torch.randn(n, n, device="cuda:0", generator=g) / math.sqrt(n)).to(dt)
        bt = b.t().contiguous()
        for lay, f in (("NN", lambda: a @ b), ("TN", lambda: a @ bt.t())):
            warm(torch, lambda i: f())
            med = batch_ms(torch, stream, lambda i: f(), max(steps, 20))
            out[f"{name}_{n}_{lay}"] = {"ms": round(med, 4), "tflops": round(2.0 * n ** 3 / (med * 1e-3) / 1e12, 1)}
    # the shapes of the `shapes` leg, row-major a @ b (hipBLAS NN)
    for name, dt, m, nn, k in (("fp32_3072", torch.float32, 3072, 3072, 3072),
                               ("fp32_5120", torch.float32, 5120, 5120, 5120),
                               ("fp32_4000x4000x4096", torch.float32, 4000, 4000, 4096),
                               ("fp16_3072", torch.float16, 3072, 3072, 3072),
                               ("fp16_6144", torch.float16, 6144, 6144, 6144),
                               ("fp16_2047x14336x4096", torch.float16, 2047, 14336, 4096)):
        a = (torch.randn(m, k, device="cuda:0", generator=g) / math.sqrt(k)).to(dt)
        b = (torch.randn(k, nn, device="cuda:0", generator=g) / math.sqrt(k)).to(dt)
        warm(torch, lambda i: a @ b)
        med = batch_ms(torch, stream, lambda i: a @ b, max(steps, 10))
        out[f"{name}_NN"] = {"ms": round(med, 4), "tflops": round(2.0 * m * nn * k / (med * 1e-3) / 1e12, 1)}
        del a, b
    K = O = 8192
    Ws = [(torch.randn(O, K, device="cuda:0", generator=g) * 0.02).half() for _ in range(3)]
    X = torch.randn(64, K, device="cuda:0", generator=g).half()
    for nt in (1, 4, 8, 16, 24, 32, 64):
        x = X[:nt]
        warm(torch, lambda i: x @ Ws[i % 3].t())
        med = batch_ms(torch, stream, lambda i: x @ Ws[i % 3].t(), 3 * max(steps, 10))
        nbytes = 2 * O * K + 2 * K * nt + 2 * O * nt
        out[f"decode_8192_n{nt}"] = {"us": round(med * 1e3, 2), "GBps": round(nbytes / (med * 1e-3) / 1e9, 1)}
    # x @ w with w stored K x O (row-major [K, O], hipBLAS NN)
    Wk = [w.t().contiguous() for w in Ws]
    del Ws
    for nt in (1, 8, 16, 32):
        x = X[:nt]
        warm(torch, lambda i: x @ Wk[i % 3])
        med = batch_ms(torch, stream, lambda i: x @ Wk[i % 3], 3 * max(steps, 10))
        nbytes = 2 * O * K + 2 * K * nt + 2 * O * nt
        out[f"decodeKxO_8192_n{nt}"] = {"us": round(med * 1e3, 2), "GBps": round(nbytes / (med * 1e-3) / 1e9, 1)}
    return out


def batched(torch, vk, stream, steps):
    """configs[4] second half: strided-batched fp32, batch 64 of 512^3 (NN)."""
    sp = stream.cuda_stream
    n, nb = 512, 64
    g = torch.Generator(device="cuda:0").manual_seed(64)
    A = torch.rand(nb * n * n, device="cuda:0", generator=g) * 2 - 1     # U[-1, 1)
    B = torch.rand(nb * n * n, device="cuda:0", generator=g) * 2 - 1
    C = torch.empty(nb * n * n, device="cuda:0")

    def call():
        vk.gemm_async(vk.DT_F32, vk.DT_F32, 0, 0, n, n, n, 1.0, B.data_ptr(), n, A.data_ptr(), n, 0.0, C.data_ptr(),
                      n, nb, n * n, n * n, n * n, stream=sp)
    warm(torch, lambda i: call())
    med = batch_ms(torch, stream, lambda i: call(), max(steps, 20))
    tf = 2.0 * nb * n ** 3 / (med * 1e-3) / 1e12
    return {"ms": round(med, 4), "tflops": round(tf, 2), "frac_of_peak": round(tf / PEAK_FP32_TFLOPS, 4),
            "path": vk.PATH_NAMES[vk.last_path()]}


if __name__ == "__main__":
    main()
