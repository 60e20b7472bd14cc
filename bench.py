#!/usr/bin/env python3
"""Benchmark of the quantized-linear hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--no-cpu]

Workload: greedy decode of a random-init Qwen2-0.5B-shaped int4 GPTQ model (24 layers, hidden
896, 14/2 heads of 64, intermediate 4864, vocab 151936, group size 128, tied head re-quantized
on the device) with the library's decode engine. A "step" is one decode token: one replay of
the captured graph (embedding, 24 layers, head GEMV, device argmax), after a 64-token prefill.
The weights (synthetic, seeded) are in HBM before timing.

The step is one launch of the persistent decode kernel (the engine's default where the shape
allows it). The JSON line reports `value` = algorithmic bytes of the step's int4 GEMVs (every
weight of the model once per token) / step time, in GB/s, plus decode tokens/s and the same
step as a launch sequence; `roofline` for the persistent kernel (its algorithmic bytes: weights,
activations, KV rows, over its launch time); the drop-in GEMV kernel on the token's 97 GEMVs
replayed alone over two alternating weight copies (522 MB, above the 256 MB Infinity Cache, so
from HBM), with per-shape timings; the GGUF Q4_K GEMV (Llama-3-8B up_proj), the act-order
prefill GEMM (K = N = 4096) and the Qwen3-MoE expert block; and `cpu_baseline`: the
reference's numpy fallback (restated in `oracle/`) timed on this host on a bounded sample of
the same GEMVs.
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
H, NH, NKV, HD, I, V, LAYERS, GS = 896, 14, 2, 64, 4864, 151936, 24, 128  # Qwen2-0.5B
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


def timed(torch, fn, reps, warm=1, min_warm_s=0.03, min_timed_s=0.02):
    """Seconds per call of fn (GPU time between events). The GPU is first kept busy for at
    least min_warm_s (its clocks ramp up under load; a cold first measurement reads slow), and
    the timed window is stretched to at least min_timed_s."""
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0, n = time.perf_counter(), 0
    while n < warm or time.perf_counter() - t0 < min_warm_s:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    s.record()
    fn()
    e.record()
    e.synchronize()
    per = max(s.elapsed_time(e) * 1e-3, 1e-7)
    reps = max(reps, int(min_timed_s / per) + 1)
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


def ggml_bench(torch, core, type_name, copies=12, reps=24):
    """GGUF Q8_0 / Q6_K GEMV at the Llama-3-8B up_proj shape: x fp16 (1, 4096) -> y fp32
    (1, 14336), over `copies` distinct weight copies (above the 256 MB Infinity Cache)."""
    K, N = 4096, 14336
    vals, blk = {"Q8_0": (32, 34), "Q6_K": (256, 210)}[type_name]
    nb = N * K // vals
    w = torch.randint(0, 256, (copies, nb, blk), dtype=torch.uint8, device="cuda")
    d = 0 if type_name == "Q8_0" else 208
    w[:, :, d + 1] &= 0x3B  # finite fp16 d
    w = w.reshape(copies, N, -1)
    x = torch.randn((1, K), device="cuda").half()
    out = torch.empty((1, N), device="cuda")

    def run():
        for i in range(reps):
            core.ggml_matmul(x, w[i % copies], type_name, K, N, out=out)
    run()
    torch.cuda.synchronize()
    g = capture(torch, run)
    t = timed(torch, g.replay, 5) / reps
    nbytes = nb * blk + K * 2 + N * 4
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


def moe_bench(torch, core, reps=8):
    """Qwen3-MoE block: T=256 tokens of hidden 2048, 128 experts (gate/up 2048->768, down
    768->2048, int4 gs=128), top-8; routing + grouped GEMMs + combine on the device."""
    from webpytorch_amd import synth
    w = synth.moe_workload(3)
    ex = core.MoEExperts(w["experts"])
    x = torch.from_numpy(w["x"]).cuda()
    lg = torch.from_numpy(w["logits"]).cuda()

    def run():
        for _ in range(reps):
            ex(x, lg, 8)
    run()
    torch.cuda.synchronize()
    g = capture(torch, run)
    t = timed(torch, g.replay, 5) / reps
    nbytes = 128 * 3 * gemv_bytes(2048, 768, "f16", False)
    flops = 256 * 8 * 2 * (2 * 2048 * 768 + 768 * 2048)
    del g
    return {"us": round(t * 1e6, 2), "weight_GBs": round(nbytes / t / 1e9, 1),
            "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4), "TFLOPs": round(flops / t / 1e12, 1)}


def gemv_large(torch, core, reps=24):
    """The GEMV operator on bandwidth-bound 7B-class shapes (int4, gs 128, fp16 scales, 1 row of
    fp16 or fp32 activations), over enough distinct weight copies (>= 600 MB) that every launch
    reads HBM: GB/s of algorithmic bytes and the fraction of the 8 TB/s peak."""
    res = {}
    for name, K, N, xdt in (("llama7b_up_4096x11008_f16x", 4096, 11008, torch.float16),
                            ("llama7b_down_11008x4096_f16x", 11008, 4096, torch.float16),
                            ("llama7b_up_4096x11008_f32x", 4096, 11008, torch.float32)):
        nb = gemv_bytes(K, N, "f16", False) + (K * 2 if xdt == torch.float32 else 0)
        copies = max(2, int(600e6 // nb) + 1)
        ws = [make_layer(torch, K, N, "f16", False) for _ in range(copies)]
        x = torch.randn((1, K), device="cuda").to(xdt)
        y = torch.empty((1, N), device="cuda", dtype=torch.float16)

        def run(ws=ws, x=x, y=y, K=K, N=N):
            for i in range(reps):
                qw, qz, sc, _ = ws[i % len(ws)]
                core._gptq_matmul(x, qw, qz, sc, K, N, GS, 4, 1.0, out=y)
        run()
        torch.cuda.synchronize()
        g = capture(torch, run)
        t = timed(torch, g.replay, 5) / reps
        res[name] = {"bytes": nb, "us": round(t * 1e6, 3), "GBs": round(nb / t / 1e9, 1),
                     "frac": round(nb / t / 1e9 / HBM_PEAK_GBS, 4)}
        del g, ws
        torch.cuda.empty_cache()
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


def gemv_only(torch, core, steps):
    """The step's 97 int4 GEMVs alone (no other kernels), over two alternating weight copies:
    the roofline measurement of the GEMV kernel, and per-shape timings."""
    copies = []
    for c in range(2):
        layers = [{k: make_layer(torch, K, N, sdt, b) for k, (K, N, sdt, _, b) in SHAPES.items() if k != "head"}
                  for _ in range(LAYERS)]
        K, N, sdt, _, b = SHAPES["head"]
        copies.append((layers, make_layer(torch, K, N, sdt, b)))
    xs = {k: torch.randn((1, K), device="cuda") for k, (K, *_r) in SHAPES.items()}
    ys = {k: torch.empty((1, N), device="cuda") for k, (K, N, *_r) in SHAPES.items()}

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
    for c in range(2):
        step(c)
    torch.cuda.synchronize()
    graphs = [capture(torch, lambda c=c: step(c)) for c in range(2)]
    for i in range(4):
        graphs[i % 2].replay()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(steps):
        graphs[i % 2].replay()
    ev1.record()
    ev1.synchronize()
    t = ev0.elapsed_time(ev1) * 1e-3 / steps
    del graphs
    kernels = {}
    for name, (K, N, sdt, zoff, b) in SHAPES.items():
        ws = [copies[c][0][l][name] for c in range(2) for l in range(LAYERS)] if name != "head" else \
            [copies[c][1] for c in range(2)]
        reps = 48 if name != "head" else 16

        def run(name=name, ws=ws, reps=reps):
            for i in range(reps):
                gemv(name, ws[i % len(ws)])
        g = capture(torch, run)
        tt = timed(torch, g.replay, 5) / reps
        nb = gemv_bytes(K, N, sdt, b)
        kernels[name] = {"K": K, "N": N, "bytes": nb, "us": round(tt * 1e6, 3), "GBs": round(nb / tt / 1e9, 1)}
        del g
    return t, kernels


def decode_step_time(torch, m, ids, warmup, steps):
    """Prefill + one step (which captures the decode graph), `warmup` untimed replays, then the
    mean time of `steps` replays between events on the replay stream."""
    r = m.generate(ids, 2)
    pos0 = int(m.state[0])
    g = m._graph
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(steps):
        g.replay()
    ev1.record(stream)
    ev1.synchronize()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) * 1e-3 / steps, r, pos0


def copy_calibration(torch, nbytes=1 << 30, reps=2):
    """A plain streaming kernel over `nbytes` (torch's fp32 elementwise add, ordinary cached
    loads and stores), `reps` times, from a source that a 1 GiB write has pushed out of the 256 MB
    Infinity Cache: reads and writes exactly `nbytes` from and to HBM each time, the scale for the
    FETCH_SIZE / WRITE_SIZE counters. (The runtime's own copy kernel reads in a way these
    counters do not see.)"""
    src = torch.rand(nbytes // 4, device="cuda")
    dst = torch.empty_like(src)
    evict = torch.empty(1 << 28, device="cuda")
    for _ in range(reps):
        evict.fill_(1.0)
        torch.add(src, 1.0, out=dst)
    torch.cuda.synchronize()
    del evict
    return nbytes


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_persistent_hbm_traffic_qwen2_05b_int4.md")


def measured_traffic():
    """HBM bytes per launch of the persistent decode kernel, from the committed FETCH_SIZE /
    WRITE_SIZE counter summary (its `traffic_bytes_per_launch:` line), or None if it is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":")[1]))
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-extras", action="store_true", help="only the decode step and its roofline")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the token's GEMVs alone and a plain 1 GiB copy, for hardware-counter runs")
    ap.add_argument("--gemv-large", action="store_true", help="only the GEMV operator on 7B-class shapes")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the persistent decode step and a plain 1 GiB copy, for hardware-counter runs")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the quantized-linear path has no multi-GPU mode here "
              "(column/expert sharding is a design note only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from webpytorch_amd import core, llm, synth
    torch.cuda.set_device(0)
    torch.manual_seed(0)
    if a.gemv_large:
        print(json.dumps(gemv_large(torch, core)), flush=True)
        return
    if a.decode_only:
        m = llm.CausalLM.from_weights(synth.decoder_weights(5, **synth.QWEN2_05B), lmax=256)
        t, _, _ = decode_step_time(torch, m, synth.prompt_ids(5, 64, synth.QWEN2_05B["V"]), 2, a.steps)
        copy_bytes = copy_calibration(torch)
        print(json.dumps({"decode_step_us": round(t * 1e6, 2), "copy_bytes_read": copy_bytes,
                          "copy_bytes_written": copy_bytes, "error_bits": m.persistent_error()}), flush=True)
        return
    if a.gemv_only:
        t_gemv, kernels = gemv_only(torch, core, a.steps)
        copy_bytes = copy_calibration(torch)
        print(json.dumps({"gemv_step_us": round(t_gemv * 1e6, 2), "gemv_shapes": kernels,
                          "copy_bytes_read": copy_bytes, "copy_bytes_written": copy_bytes}), flush=True)
        return

    prompt = 64
    lmax = max(256, prompt + a.warmup + a.steps + 2)
    w = synth.decoder_weights(5, **synth.QWEN2_05B)
    ids = synth.prompt_ids(5, prompt, synth.QWEN2_05B["V"])
    m = llm.CausalLM.from_weights(w, lmax=lmax)
    if m.pws is None:
        raise SystemExit("the persistent decode step is not available for this shape")
    t_step, r, pos0 = decode_step_time(torch, m, ids, a.warmup, a.steps)
    if m.persistent_error():
        raise SystemExit("persistent decode step reported error bits %d" % m.persistent_error())
    step_bytes = sum(LAYERS * gemv_bytes(K, N, sdt, b) for k, (K, N, sdt, _, b) in SHAPES.items() if k != "head")
    step_bytes += gemv_bytes(*[SHAPES["head"][i] for i in (0, 1, 2, 4)])
    value = step_bytes / t_step / 1e9
    # the kernel's algorithmic bytes: weights, activations, the KV rows of positions 0..pos (read)
    # and pos (written) over 24 layers x 2 kv heads x (k, v), the embedding row
    pos_mid = pos0 + (a.warmup + a.steps) / 2.0
    kv_bytes = int(LAYERS * NKV * 2 * HD * 4 * (pos_mid + 2))
    kernel_bytes = step_bytes + kv_bytes + H * 2
    achieved = kernel_bytes / t_step / 1e9

    # the same step as a launch sequence (5 launches per layer + head + argmax), for comparison
    del m
    torch.cuda.empty_cache()
    ms = llm.CausalLM.from_weights(w, lmax=lmax, persistent=False)
    t_seq, _, _ = decode_step_time(torch, ms, ids, a.warmup, a.steps)
    del ms
    torch.cuda.empty_cache()

    t_gemv, kernels = gemv_only(torch, core, a.steps)
    launches = LAYERS * 4 + 1
    res = {
        "metric": "int4 GEMV achieved HBM GB/s (% of peak) + decode tokens/s, Qwen2-0.5B shape",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(t_step * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int4 weights, fp32 activations, fp32 accumulate", "data": "synthetic",
        "config": {"workload": "greedy decode, random-init Qwen2-0.5B-shaped int4 GPTQ model (24 layers, "
                               "hidden 896, 14/2 heads, intermediate 4864, vocab 151936, gs=128), 64-token "
                               "prompt; one step = one decode token = one launch of the persistent decode "
                               "kernel (captured graph replay)",
                   "gemv_bytes_per_token": step_bytes, "kernel_bytes_per_token": kernel_bytes,
                   "launches_per_token": 1},
        "decode_tokens_per_s": round(1.0 / t_step, 1),
        "decode_tokens_per_s_launch_sequence": round(1.0 / t_seq, 1),
        "ttft_ms": round(r.ttft_s * 1e3, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "traffic_note": "HBM bytes per launch (FETCH_SIZE + WRITE_SIZE of the kernel, scaled by "
                                     "the counters' reading for a plain copy of known size)",
                     "kernel": "miq::pd::decode_persistent_kernel",
                     "measured_on": "the timed graph replays (one launch per token)",
                     "avg_launch_us": round(t_step * 1e6, 2), "algorithmic_bytes_per_launch": kernel_bytes},
        "gemv_kernel": {"kernel": "the drop-in GEMV operator (one row of int4 codes: miq::gm::gemv_mma_kernel)",
                        "measured_on": "the token's 97 GEMVs alone, 2 alternating weight copies (522 MB)",
                        "avg_launch_us": round(t_gemv / launches * 1e6, 3),
                        "achieved_GBs": round(step_bytes / t_gemv / 1e9, 2),
                        "frac": round(step_bytes / t_gemv / 1e9 / HBM_PEAK_GBS, 4), "shapes": kernels},
    }
    if not a.no_extras:
        res["gemv_large"] = gemv_large(torch, core)
        res["q4k_gemv_llama3_8b_up"] = q4k_bench(torch, core)
        res["q6k_gemv_llama3_8b_up"] = ggml_bench(torch, core, "Q6_K")
        res["q8_0_gemv_llama3_8b_up"] = ggml_bench(torch, core, "Q8_0")
        res["gptq_gemm_act_order_4096"] = gemm_bench(torch, core)
        res["moe_qwen3_t256"] = moe_bench(torch, core)
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline(a.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
