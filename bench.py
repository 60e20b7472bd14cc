#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--no-cpu]

Workload (one "step"): every int4 GPTQ GEMV of one decode token of a Qwen2-0.5B-shaped model
(hidden 896, 14/2 heads of 64, intermediate 4864, vocab 151936, group size 128), M = 1,
fp16 activations:
  24 layers x {qkv 896->1152 (+ fp32 bias), o 896->896, gate_up 896->9728, down 4864->896}
  + the tied head 896->151936 (fp32 scales, zero offset 0, as the head re-quantization makes it).
q/k/v and gate/up share their input, so each pair or triple runs as one GEMV over the
concatenated columns (per-column groups make that identical to separate layers). The weights
(random bits, synthetic) sit in HBM before timing; two distinct copies of the whole set
(~522 MB, more than the 256 MB Infinity Cache) alternate between steps so every step
streams from HBM. Each step is one HIP graph replay on the current stream.

The JSON line reports `value` = algorithmic bytes of the step's GEMVs / step time (GB/s);
`roofline` for the GEMV kernel (the only kernel of the step); per-shape timings; the GGUF
Q4_K GEMV at the Llama-3-8B up_proj shape; and `cpu_baseline`: the reference's numpy
fallback (restated in `oracle/`) timed on this host on a bounded sample of the same GEMVs.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
H, NH, NKV, HD, I, V, LAYERS, GS = 896, 14, 2, 64, 4864, 151936, 24, 128
SHAPES = {  # name: (K, N, scales dtype, zero offset, bias)
    "qkv": (H, (NH + 2 * NKV) * HD, "f16", 1.0, True),
    "o": (NH * HD, H, "f16", 1.0, False),
    "gate_up": (H, 2 * I, "f16", 1.0, False),
    "down": (I, H, "f16", 1.0, False),
    "head": (H, V, "f32", 0.0, False),
}


def gemv_bytes(K, N, sdt, bias):
    """Algorithmic HBM bytes of one M=1 int4 GEMV: packed codes, zeros, scales, bias, x, y."""
    return (K // 8) * N * 4 + (K // GS) * (N // 8) * 4 + (K // GS) * N * (2 if sdt == "f16" else 4) + \
        (N * 4 if bias else 0) + K * 2 + N * 2


def make_layer(torch, K, N, sdt, bias):
    dev = "cuda"
    qw = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), dtype=torch.int32, device=dev)
    qz = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // GS, N // 8), dtype=torch.int32, device=dev)
    sc = torch.rand((K // GS, N), device=dev) * 0.01 + 1e-3
    sc = sc.half() if sdt == "f16" else sc
    b = (torch.randn(N, device=dev) * 0.02) if bias else None
    return qw, qz, sc, b


def timed(torch, fn, reps, warm=1):
    for _ in range(warm):
        fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) * 1e-3 / reps


def capture(torch, fn):
    """Record fn's launches (already warmed up eagerly) into a HIP graph."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def q4k_bench(torch, core, copies=16, reps=32):
    """GGUF Q4_K GEMV, Llama-3-8B up_proj: x fp16 (1, 4096) -> y fp32 (1, 14336)."""
    K, N = 4096, 14336
    nb = N * K // 256
    w = torch.randint(0, 256, (copies, nb, 144), dtype=torch.uint8, device="cuda")
    w[:, :, 1] &= 0x3B  # finite fp16 d and dmin
    w[:, :, 3] &= 0x3B
    w = w.reshape(copies, N, -1)
    x = torch.randn((1, K), device="cuda").half()
    out = torch.empty((1, N), device="cuda")

    def run():
        for i in range(reps):
            core.ggml_matmul(x, w[i % copies], "Q4_K", K, N, out=out)
    run()
    torch.cuda.synchronize()
    g = capture(torch, run)
    t = timed(torch, g.replay, 5) / reps
    nbytes = nb * 144 + K * 2 + N * 4
    return {"K": K, "N": N, "bytes": nbytes, "us": round(t * 1e6, 3), "GBs": round(nbytes / t / 1e9, 1),
            "frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}


MFMA_PEAK_TFLOPS = 2500.0  # dense fp16


def gemm_bench(torch, core, Ms=(16, 128, 512), copies=32, reps=32):
    """GPTQ int4 prefill GEMM, act-order (rows repacked at load), K = N = 4096, gs = 128:
    x fp16 (M, 4096) -> y fp16 (M, 4096), over `copies` distinct weight copies."""
    K = N = 4096
    perm = torch.randperm(K, device="cuda").int()
    ws = [make_layer(torch, K, N, "f16", False) for _ in range(copies)]
    res = {}
    for M in Ms:
        x = torch.randn((M, K), device="cuda").half()
        y = torch.empty((M, N), device="cuda", dtype=torch.float16)

        def run(M=M, x=x, y=y):
            for i in range(reps):
                qw, qz, sc, _ = ws[i % copies]
                core._gptq_matmul(x, qw, qz, sc, K, N, GS, 4, 1.0, perm=perm, out=y)
        run()
        torch.cuda.synchronize()
        g = capture(torch, run)
        t = timed(torch, g.replay, 5) / reps
        flops = 2.0 * M * K * N
        nbytes = gemv_bytes(K, N, "f16", False) - K * 2 - N * 2 + 2 * M * K * 2
        res["M%d" % M] = {"us": round(t * 1e6, 3), "TFLOPs": round(flops / t / 1e12, 1),
                          "mfma_frac": round(flops / t / 1e12 / MFMA_PEAK_TFLOPS, 4),
                          "GBs": round(nbytes / t / 1e9, 1), "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}
        del g
    return res


def cpu_baseline(seconds=10.0):
    """The reference's numpy-fallback GEMV path (`_gptq_matmul_np`, restated in oracle/) on a
    bounded sample: one decoder layer's seven linears (q, k, v, o, gate, up, down as separate
    layers, as the reference holds them) plus four 4096-row head blocks, repeated for about
    `seconds`; throughput in the same algorithmic bytes as the GPU figure."""
    import numpy as np
    from oracle import gptq
    from webpytorch_amd import synth
    lin = [("q", H, NH * HD, np.float16, 1.0), ("k", H, NKV * HD, np.float16, 1.0),
           ("v", H, NKV * HD, np.float16, 1.0), ("o", NH * HD, H, np.float16, 1.0),
           ("gate", H, I, np.float16, 1.0), ("up", H, I, np.float16, 1.0), ("down", I, H, np.float16, 1.0)]
    lin += [("head%d" % i, H, 4096, np.float32, 0.0) for i in range(4)]
    layers = []
    nbytes = 0
    for name, K, N, sdt, zoff in lin:
        L = synth.gptq_layer(17, K, N, GS, 4, name=name)
        L["scales"] = L["scales"].astype(sdt)
        x = synth.activations(17, 1, K, np.float16, name="x" + name).astype(np.float32)
        layers.append((L, x, zoff))
        nbytes += gemv_bytes(K, N, "f16" if sdt == np.float16 else "f32", name in ("q", "k", "v"))

    def one():
        for L, x, zoff in layers:
            gptq.gptq_matmul_np(x, L["qweight"], L["qzeros"], L["scales"], L["K"], L["N"], GS, 4, zoff)
    one()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    t = float(np.median(times))
    try:
        from threadpoolctl import threadpool_info
        cores = max([p.get("num_threads", 1) for p in threadpool_info()] or [1])
    except Exception:
        cores = len(os.sched_getaffinity(0))
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": int(cores), "kind": "port",
            "sample": "numpy restatement of _gptq_matmul_np: 1 Qwen2-0.5B layer (7 linears) + 4 head "
                      "blocks of 4096 rows, %d reps, median %.1f ms, %d algorithmic bytes" % (
                          len(times), t * 1e3, nbytes)}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the quantized-linear path has no multi-GPU mode here "
              "(column/expert sharding is a design note only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from webpytorch_amd import core
    torch.cuda.set_device(0)
    torch.manual_seed(0)

    copies = []
    for c in range(2):
        layers = [{k: make_layer(torch, K, N, sdt, b) for k, (K, N, sdt, _, b) in SHAPES.items() if k != "head"}
                  for _ in range(LAYERS)]
        K, N, sdt, _, b = SHAPES["head"]
        copies.append((layers, make_layer(torch, K, N, sdt, b)))
    xs = {k: torch.randn((1, K), device="cuda").half() for k, (K, *_r) in SHAPES.items()}
    ys = {k: torch.empty((1, N), device="cuda", dtype=torch.float16) for k, (K, N, *_r) in SHAPES.items()}

    def gemv(name, w):
        K, N, sdt, zoff, _ = SHAPES[name]
        qw, qz, sc, b = w
        core._gptq_matmul(xs[name], qw, qz, sc, K, N, GS, 4, zoff, bias=b, out=ys[name])

    def step(c):
        layers, head = copies[c]
        for lay in layers:
            for name in ("qkv", "o", "gate_up", "down"):
                gemv(name, lay[name])
        gemv("head", head)

    launches = LAYERS * 4 + 1
    step_bytes = sum(LAYERS * gemv_bytes(K, N, sdt, b) for k, (K, N, sdt, _, b) in SHAPES.items() if k != "head")
    step_bytes += gemv_bytes(*[SHAPES["head"][i] for i in (0, 1, 2, 4)])
    for c in range(2):
        step(c)
    torch.cuda.synchronize()
    graphs = [capture(torch, lambda c=c: step(c)) for c in range(2)]

    for i in range(a.warmup):
        graphs[i % 2].replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(a.steps):
        graphs[i % 2].replay()
    ev1.record(stream)
    ev1.synchronize()
    torch.cuda.synchronize()
    t_step = ev0.elapsed_time(ev1) * 1e-3 / a.steps
    value = step_bytes / t_step / 1e9
    per_launch = t_step / launches

    # per-shape sustained time: graphs of back-to-back launches of one shape over 48 copies
    kernels = {}
    for name, (K, N, sdt, zoff, b) in SHAPES.items():
        ws = [copies[c][0][l][name] for c in range(2) for l in range(LAYERS)] if name != "head" else \
            [copies[c][1] for c in range(2)]
        reps = 48 if name != "head" else 16

        def run(name=name, ws=ws, reps=reps):
            for i in range(reps):
                gemv(name, ws[i % len(ws)])
        g = capture(torch, run)
        t = timed(torch, g.replay, 5) / reps
        nb = gemv_bytes(K, N, sdt, b)
        kernels[name] = {"K": K, "N": N, "bytes": nb, "us": round(t * 1e6, 3), "GBs": round(nb / t / 1e9, 1)}
        del g
    q4k = q4k_bench(torch, core)
    gemm = gemm_bench(torch, core)

    res = {
        "metric": "int4 GEMV achieved HBM GB/s (% of peak) + decode tokens/s, Qwen2-0.5B shape",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(t_step * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int4 weights, fp16 activations, fp32 accumulate", "data": "synthetic",
        "config": {"workload": "Qwen2-0.5B int4 GPTQ decode-step GEMVs, M=1: 24 x {qkv 896->1152, "
                               "o 896->896, gate_up 896->9728, down 4864->896} + head 896->151936; gs=128; "
                               "2 alternating weight copies (522 MB)",
                   "launches_per_step": launches, "bytes_per_step": step_bytes},
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "miq::gptq_gemv_kernel", "avg_launch_us": round(per_launch * 1e6, 3),
                     "avg_bytes_per_launch": step_bytes // launches},
        "gemv_shapes": kernels,
        "q4k_gemv_llama3_8b_up": q4k,
        "gptq_gemm_act_order_4096": gemm,
    }
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline(a.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
