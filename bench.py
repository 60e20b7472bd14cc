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
from HBM), with per-shape timings; config 0 exactly (fp16 in and out, 256 launches over distinct
copies, plus single-launch latency); the full 128-token decode of the end-to-end config; the GGUF
Q4_K GEMV (Llama-3-8B up_proj) and its prefill GEMM (M = 64 and 512), the act-order prefill GEMM
(K = N = 4096) in int4 and in per-channel int8, and the Qwen3-MoE expert block; and `cpu_baseline`: the reference's numpy
fallback (restated in `oracle/`) timed on this host on bounded samples of every config.
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


def ggml_gemm_bench(torch, core, type_name="Q4_K", reps=10):
    """GGUF prefill GEMM (`miq_ggml_gemm`) at the Llama-3-8B up_proj shape: x (M, 4096) fp16 or
    fp32 -> y fp32 (M, 14336) on the matrix cores, over enough distinct weight copies (>= 330 MB,
    above the 256 MB Infinity Cache) that every launch reads its weights from HBM; TFLOP/s and
    the fraction of the dense fp16 peak."""
    K, N = 4096, 14336
    vals, blk = {"Q4_K": (256, 144), "Q5_K": (256, 176), "Q6_K": (256, 210), "Q8_0": (32, 34)}[type_name]
    nb = N * K // vals
    copies = max(2, -(-330_000_000 // (nb * blk)))
    w = random_blocks(torch, type_name, copies, nb, blk).reshape(copies, N, -1)
    res = {"copies": copies, "weight_bytes": nb * blk}
    for M, dt in ((64, torch.float16), (512, torch.float16), (512, torch.float32)):
        x = torch.randn((M, K), device="cuda").to(dt)
        out = torch.empty((M, N), device="cuda")

        def run(x=x, out=out):
            for i in range(reps):
                core.ggml_matmul(x, w[i % copies], type_name, K, N, out=out)
        run()
        torch.cuda.synchronize()
        g = capture(torch, run)
        t = timed(torch, g.replay, 5) / reps
        del g
        flops = 2.0 * M * K * N
        res["M%d_%s" % (M, "f16" if dt == torch.float16 else "f32")] = {
            "us": round(t * 1e6, 2), "TFLOPs": round(flops / t / 1e12, 1),
            "mfma_frac": round(flops / t / 1e12 / MFMA_PEAK_TFLOPS, 4)}
    return res


def random_blocks(torch, type_name, copies, nb, blk):
    """Uniform random block bytes on the device with every fp16 scale field small and finite."""
    w = torch.randint(0, 256, (copies, nb, blk), dtype=torch.uint8, device="cuda")
    for off in {"Q4_K": (0, 2), "Q5_K": (0, 2), "Q6_K": (208,), "Q8_0": (0,)}[type_name]:
        w[:, :, off + 1] &= 0x17  # fp16 exponent field <= 5: |scale| < 2^-9
    return w


def prefill_ttft(torch, llm, core, T=64, reps=5):
    """Time to first token of a T-token prompt on a Llama-3-8B-shaped decoder whose weights stay
    in a Q4_K_M file's mix of GGUF encodings: q, k, o, gate and up in Q4_K; v and down in Q6_K on
    the layers that recipe gives more bits (the first and last eighth of the layers and every
    third one between), Q4_K elsewhere; the output head in Q6_K (random blocks; the embedding
    table as a GGUF file's decoded fp32 one).
    One prefill = embedding, 32 layers of RMSNorm, q|k|v, RoPE + KV write, attention, o, RMSNorm,
    gate|up, SwiGLU and down (the projections at T rows on the matrix cores), then the last row's
    head GEMV and arg-max."""
    L, H, NH, NKV, HD, I, V = 32, 4096, 32, 8, 128, 14336, 128256
    more_bits = lambda i: i < L // 8 or i >= 7 * L // 8 or (i - L // 8) % 3 == 2  # noqa: E731

    def lin(t, K, N):
        vals, blk = (256, 144) if t == "Q4_K" else (256, 210)
        return core.GGMLLinear(random_blocks(torch, t, 1, N * K // vals, blk).reshape(-1), t, K, N)
    layers = []
    for i in range(L):
        hi = "Q6_K" if more_bits(i) else "Q4_K"
        layers.append({"q": lin("Q4_K", H, NH * HD), "k": lin("Q4_K", H, NKV * HD), "v": lin(hi, H, NKV * HD),
                       "o": lin("Q4_K", NH * HD, H), "gate": lin("Q4_K", H, I), "up": lin("Q4_K", H, I),
                       "down": lin(hi, I, H), "in_ln": torch.ones(H), "post_ln": torch.ones(H)})
    w = {"layers": layers, "embed": torch.randn((V, H), device="cuda") * 0.02,
         "final_norm": torch.ones(H), "head_linear": lin("Q6_K", H, V),
         "cfg": dict(L=L, H=H, NH=NH, NKV=NKV, HD=HD, I=I, V=V, gs=128, bits=4, eps=1e-5, theta=500000.0)}
    m = llm.CausalLM.from_weights(w, lmax=256)
    nbytes = sum(p.packed.numel() for lay in m.layers for k in ("qkv", "o", "gate_up", "down")
                 for p in (lay[k].parts if hasattr(lay[k], "parts") else [lay[k]]))
    ids = torch.randint(0, V, (T,), dtype=torch.int32, device="cuda")
    ts = []
    for _ in range(reps + 1):
        m.reset()
        m.ids[:T].copy_(ids)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        m._step(T)
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    t = sorted(ts[1:])[len(ts[1:]) // 2]
    flops = 2.0 * T * L * (H * (NH + 2 * NKV) * HD + NH * HD * H + 3 * H * I)
    res = {"prompt_tokens": T, "ttft_ms": round(t * 1e3, 3), "prefill_tokens_per_s": round(T / t, 1),
           "layer_weight_bytes": int(nbytes), "projection_TFLOPs": round(flops / t / 1e12, 1),
           "model": "Llama-3-8B shape (32 layers, hidden 4096, 32/8 heads of 128, intermediate 14336, vocab 128256)"}
    del m, w, layers
    torch.cuda.empty_cache()
    return res


def gemm_bench(torch, core, Ms=(16, 128, 512), copies=40, reps=40):
    """GPTQ int4 prefill GEMM, act-order (rows repacked at load), K = N = 4096, gs = 128:
    x fp16 (M, 4096) -> y fp16 (M, 4096), over `copies` distinct weight copies (40 x 8.4 MB, well
    above the 256 MB Infinity Cache)."""
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
        # the vendor library's dense fp16 GEMM of the same shape (torch.matmul -> hipBLASLt), over
        # 8 distinct fp16 weight copies, as a reference point for the matrix-core fraction
        wd = [torch.randn((K, N), device="cuda").half() for _ in range(8)]

        def dense(x=x, wd=wd):
            for i in range(reps):
                torch.matmul(x, wd[i % 8])
        dense()
        torch.cuda.synchronize()
        td = timed(torch, dense, 3) / reps
        res["M%d" % M]["dense_fp16_library_us"] = round(td * 1e6, 3)
        res["M%d" % M]["dense_fp16_library_mfma_frac"] = round(flops / td / 1e12 / MFMA_PEAK_TFLOPS, 4)
        del wd
    return res


def config0_bench(torch, core, reps=256):
    """GPTQ int4 GEMV exactly as config 0: x fp16 (1, 896) -> y fp16 (1, 4864) (Qwen2-0.5B
    gate_proj, gs 128, fp16 scales, zero offset 1), R = 256 back-to-back launches in one graph over
    256 distinct weight copies (583 MB, above the 256 MB Infinity Cache, so every launch reads
    HBM): per-call time = total / R. Single-launch latency: one eager call between events (launch
    overhead included)."""
    K, N = 896, 4864
    ws = [make_layer(torch, K, N, "f16", False) for _ in range(reps)]
    x = torch.randn((1, K), device="cuda").half()
    y = torch.empty((1, N), device="cuda", dtype=torch.float16)

    def one(i=0):
        qw, qz, sc, _ = ws[i]
        core._gptq_matmul(x, qw, qz, sc, K, N, GS, 4, 1.0, out=y)

    def run():
        for i in range(reps):
            one(i)
    run()
    torch.cuda.synchronize()
    g = capture(torch, run)
    t = timed(torch, g.replay, 3) / reps
    lat = timed(torch, one, 64)
    nb = gemv_bytes(K, N, "f16", False)
    del g, ws
    torch.cuda.empty_cache()
    return {"K": K, "N": N, "x": "fp16 (1, 896)", "y": "fp16 (1, 4864)", "bytes": nb, "launches": reps,
            "us_per_call": round(t * 1e6, 3), "GBs": round(nb / t / 1e9, 1),
            "frac": round(nb / t / 1e9 / HBM_PEAK_GBS, 4), "single_launch_us": round(lat * 1e6, 3),
            "replay_floor": replay_floor(torch, nb, reps)}


def replay_floor(torch, nbytes, reps=256):
    """What R back-to-back launches in one graph cost with (almost) no work, per launch: an
    empty kernel (torch's spin kernel with 0 cycles), a one-wave 16-byte copy, and a copy of
    nbytes / 2 bytes (nbytes moved, as a GEMV of nbytes reads) over R distinct sources (above the
    Infinity Cache in total, so the reads come from HBM)."""
    def per_launch(fn):
        fn()
        torch.cuda.synchronize()
        g = capture(torch, fn)
        t = timed(torch, g.replay, 3) / reps
        del g
        return round(t * 1e6, 3)
    empty = per_launch(lambda: [torch.cuda._sleep(0) for _ in range(reps)])
    s4, d4 = torch.ones(4, device="cuda"), torch.empty(4, device="cuda")
    tiny = per_launch(lambda: [d4.copy_(s4) for _ in range(reps)])
    n = nbytes // 2 // 4
    srcs = torch.ones((reps, n), device="cuda")
    dst = torch.empty(n, device="cuda")
    copy = per_launch(lambda: [dst.copy_(srcs[i]) for i in range(reps)])
    del srcs
    torch.cuda.empty_cache()
    return {"empty_kernel_us": empty, "copy_16B_us": tiny, "copy_us": copy, "copy_bytes_moved": 2 * n * 4,
            "kernels": "torch spin kernel (0 cycles); torch elementwise copy"}


def gemm_int8_bench(torch, core, Ms=(16, 128, 512), copies=24, reps=24):
    """The config-2 layer quantized per output channel to symmetric int8 (dtype="int8": one
    group spanning K, stored code q + 128, zero offset 1), K = N = 4096: x fp16 (M, 4096) ->
    y fp16, over `copies` distinct weight copies."""
    K = N = 4096
    ws = []
    for _ in range(copies):
        qw = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 4, N), dtype=torch.int32, device="cuda")
        qz = torch.full((1, N // 4), 0x7F7F7F7F, dtype=torch.int32, device="cuda")
        sc = (torch.rand((1, N), device="cuda") * 0.01 + 1e-3).half()
        ws.append((qw, qz, sc))
    res = {}
    for M in Ms:
        x = torch.randn((M, K), device="cuda").half()
        y = torch.empty((M, N), device="cuda", dtype=torch.float16)

        def run(x=x, y=y):
            for i in range(reps):
                qw, qz, sc = ws[i % copies]
                core._gptq_matmul(x, qw, qz, sc, K, N, K, 8, 1.0, out=y)
        run()
        torch.cuda.synchronize()
        g = capture(torch, run)
        t = timed(torch, g.replay, 5) / reps
        flops = 2.0 * M * K * N
        nbytes = K * N + N // 4 * 4 + N * 2 + 2 * M * K * 2
        res["M%d" % M] = {"us": round(t * 1e6, 3), "TFLOPs": round(flops / t / 1e12, 1),
                          "mfma_frac": round(flops / t / 1e12 / MFMA_PEAK_TFLOPS, 4),
                          "GBs": round(nbytes / t / 1e9, 1), "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}
        del g
    return res


def decode_full(torch, m, ids, max_new=128):
    """The end-to-end config as a whole: prefill of the 64-token prompt (TTFT) and 128 greedy
    tokens (127 graph-replayed decode steps over positions 64..190), timed on the host around
    the engine's `generate` (second run: the graph is already captured)."""
    m.generate(ids, max_new)
    r = m.generate(ids, max_new)
    return {"tokens": max_new, "ttft_ms": round(r.ttft_s * 1e3, 3), "decode_tokens_per_s": round(r.decode_tok_s, 1),
            "ms_per_token": round(1e3 / r.decode_tok_s, 4) if r.decode_tok_s else None}


QWEN25_7B = dict(L=28, H=3584, NH=28, NKV=4, HD=128, I=18944, V=152064)


def device_decoder(torch, L, H, NH, NKV, HD, I, V, gs=GS, seed=7):
    """Random-init int4 GPTQ decoder of the given shape built directly in device memory (uniform
    codes and zeros, small fp16 scales so that the residual stream stays finite over the
    layers, fp16 q/k/v biases, fp32 embedding; the head is tied and quantized on load)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)

    def lin(K, N, bias=False):
        d = {"qweight": torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), dtype=torch.int32, device="cuda", generator=g),
             "qzeros": torch.randint(-2 ** 31, 2 ** 31 - 1, (K // gs, N // 8), dtype=torch.int32, device="cuda",
                                     generator=g),
             "scales": (torch.rand((K // gs, N), device="cuda", generator=g) * 0.002 + 0.0005).half()}
        if bias:
            d["bias"] = (torch.randn(N, device="cuda", generator=g) * 0.02).half()
        return d

    def vec(n):
        return (1.0 + 0.02 * torch.randn(n, device="cuda", generator=g)).float()

    layers = [{"q": lin(H, NH * HD, True), "k": lin(H, NKV * HD, True), "v": lin(H, NKV * HD, True),
               "o": lin(NH * HD, H), "gate": lin(H, I), "up": lin(H, I), "down": lin(I, H),
               "in_ln": vec(H), "post_ln": vec(H)} for _ in range(L)]
    embed = torch.randn((V, H), device="cuda", generator=g) * 0.02
    cfg = dict(L=L, H=H, NH=NH, NKV=NKV, HD=HD, I=I, V=V, gs=gs, bits=4)
    return {"layers": layers, "embed": embed, "final_norm": vec(H), "cfg": cfg}


def decode_7b(torch, llm, prompt=64, max_new=128):
    """Greedy decode of a random-init Qwen2.5-7B-shaped int4 model (28 layers, hidden 3584,
    28/4 heads of 128, intermediate 18944, vocab 152064; the shape of the reference's own
    published capture-replay figure): a 64-token prompt and 128 tokens through the engine's
    captured launch sequence (the persistent step covers hidden sizes up to 1024), timed on the
    host around `generate` (second run). Reports the weight bytes streamed per token over the
    decode time as GB/s."""
    c = QWEN25_7B
    w = device_decoder(torch, **c)
    m = llm.CausalLM.from_weights(w, lmax=prompt + max_new + 2)
    del w
    ids = torch.randint(0, c["V"], (prompt,), generator=torch.Generator().manual_seed(7)).numpy()
    m.generate(ids, max_new)
    r = m.generate(ids, max_new)
    finite = bool(torch.isfinite(m.buf["logits"]).all())
    lb = [m.head] + [lay[k] for lay in m.layers for k in ("qkv", "o", "gate_up", "down")]
    wbytes = sum(q.qweight.numel() * 4 + q.qzeros.numel() * 4 + q.scales.numel() * q.scales.element_size() +
                 (q.bias.numel() * 4 if q.bias is not None else 0) for q in lb)
    del m
    torch.cuda.empty_cache()
    return {"tokens": max_new, "ttft_ms": round(r.ttft_s * 1e3, 2), "decode_tokens_per_s": round(r.decode_tok_s, 1),
            "ms_per_token": round(1e3 / r.decode_tok_s, 3), "weight_bytes_per_token": wbytes,
            "weight_GBs": round(wbytes * r.decode_tok_s / 1e9, 1),
            "hbm_frac": round(wbytes * r.decode_tok_s / 1e9 / HBM_PEAK_GBS, 4), "finite_logits": finite,
            "path": "captured launch sequence"}


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


def _median_time(fn, seconds, min_reps=3):
    import numpy as np
    fn()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < min_reps:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def _blas_info():
    """(threads the BLAS uses, its name) from threadpoolctl / numpy's build config."""
    try:
        from threadpoolctl import threadpool_info
        info = [p for p in threadpool_info() if p.get("user_api") == "blas"]
        if info:
            return int(info[0].get("num_threads", 1)), "%s %s" % (info[0].get("internal_api", "?"),
                                                                  info[0].get("version", ""))
    except Exception:
        pass
    return len(os.sched_getaffinity(0)), "unknown"


def cpu_baseline(seconds=10.0):
    """The reference's numpy-fallback path (restated in oracle/) on bounded samples of each
    workload, on this host's cores:

    * value (the headline unit, GB/s of int4 GEMV bytes): `_gptq_matmul_np` over one decoder
      layer's seven linears (q, k, v, o, gate, up, down as separate layers, as the reference
      holds them) plus four 4096-row head blocks, all BLAS threads, and again with one thread;
    * config 1: Q4_K dequant (`ggufload.dequant`) + x @ W.T on a 1792-row band of the
      Llama-3-8B up_proj (1/8 of it);
    * config 2: `_gptq_matmul_np` at M = 128, K = N = 4096 (act-order folded into the rows);
    * config 3: `moe_mlp` at T = 32 tokens of the Qwen3-MoE block (1/8 of the 256);
    * config 4: one greedy decode step of the Qwen2-0.5B-shaped model after a one-token prompt.
    """
    import numpy as np
    from oracle import decode as odecode, gptq, moe as omoe, q4k
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

    def gemv_sample():
        for L, x, zoff in layers:
            gptq.gptq_matmul_np(x, L["qweight"], L["qzeros"], L["scales"], L["K"], L["N"], GS, 4, zoff)
    cores, blas = _blas_info()
    t, n = _median_time(gemv_sample, seconds)
    one = None
    try:
        from threadpoolctl import threadpool_limits
        with threadpool_limits(1):
            t1, _ = _median_time(gemv_sample, seconds / 4)
        one = round(nbytes / t1 / 1e9, 4)
    except Exception:
        pass
    cfg = {}
    # config 1: a 1792-row band of the Q4_K up_proj
    Kq, Nq = 4096, 1792
    Wq = synth.q4k_layer(1, Kq, Nq)
    xq = synth.activations(1, 1, Kq, np.float16)
    tq, _ = _median_time(lambda: q4k.q4k_matmul(xq, Wq, Kq, Nq), seconds / 4)
    qb = Nq * Kq // 256 * 144 + Kq * 2 + Nq * 4
    cfg["q4k_gemv"] = {"GBs": round(qb / tq / 1e9, 4), "sample": "4096 x 1792 band (1/8 of 14336 rows)"}
    # config 2: M = 128
    L2 = synth.gptq_layer(2, 4096, 4096, GS, 4)
    x2 = synth.activations(2, 128, 4096, np.float16)
    t2, _ = _median_time(lambda: gptq.gptq_matmul_np(x2, L2["qweight"], L2["qzeros"], L2["scales"], 4096, 4096, GS, 4,
                                                     1.0), seconds / 4)
    cfg["gptq_gemm_m128"] = {"TFLOPs": round(2 * 128 * 4096 * 4096 / t2 / 1e12, 5), "ms": round(t2 * 1e3, 2)}
    # config 3: 32 tokens of the MoE block
    w3 = synth.moe_workload(3)
    ex3 = [omoe.gptq_expert(e) for e in w3["experts"]]
    t3, _ = _median_time(lambda: omoe.moe_mlp_np(w3["x"][:32], w3["logits"][:32], ex3, 8), seconds / 4, 2)
    cfg["moe_t32"] = {"ms": round(t3 * 1e3, 1), "tokens_per_s": round(32 / t3, 2)}
    # config 4: one decode step (single-token prompt, then one step)
    w4 = synth.decoder_weights(5, **synth.QWEN2_05B)
    o = odecode.Qwen2Oracle(w4, lmax=8)
    cache = [None] * o.L
    nxt, _ = o.forward([1], 0, cache)
    t0 = time.perf_counter()
    o.forward([nxt], 1, cache)
    t4 = time.perf_counter() - t0
    cfg["decode_step"] = {"s_per_token": round(t4, 2), "tokens_per_s": round(1.0 / t4, 3)}
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": int(cores), "kind": "port",
            "sample": "numpy restatement of _gptq_matmul_np: 1 Qwen2-0.5B layer (7 linears) + 4 head "
                      "blocks of 4096 rows, %d reps, median %.1f ms, %d algorithmic bytes" % (n, t * 1e3, nbytes),
            "one_thread_GBs": one, "blas": blas, "host_cpus": len(os.sched_getaffinity(0)), "configs": cfg}


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
    """Prefill + one token (the first call also runs the kernels' first-use checks, so a second
    call gives the warm TTFT), `warmup` untimed decode tokens, then the mean time per token of
    `steps` decode tokens between events on the replay stream: replays of graphs of
    `m.graph_tokens` one-token steps (one persistent launch each) and one of the remainder. The
    graphs are recorded before the timed region."""
    m.generate(ids, 2)
    r = m.generate(ids, 2)
    pos0 = int(m.state[0])
    for t, _ in m._chunks(steps) + m._chunks(warmup):
        m.graph(t)
    m.replay_tokens(warmup)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    m.replay_tokens(steps)
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
    ap.add_argument("--only", choices=["gemm", "gemm_int8", "q4k", "q4k_gemm", "kq_gemm", "prefill", "moe", "config0",
                                      "decode7b", "ggml"],
                    help="one kernel benchmark and a plain 1 GiB copy, for profiler runs")
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
        out = gemv_large(torch, core)
        copy_bytes = copy_calibration(torch)
        out.update({"copy_bytes_read": copy_bytes, "copy_bytes_written": copy_bytes})
        print(json.dumps(out), flush=True)
        return
    if a.only:
        fn = {"gemm": lambda: gemm_bench(torch, core, Ms=(512,)), "gemm_int8": lambda: gemm_int8_bench(torch, core),
              "q4k": lambda: q4k_bench(torch, core), "q4k_gemm": lambda: ggml_gemm_bench(torch, core, "Q4_K"),
              "kq_gemm": lambda: {t: ggml_gemm_bench(torch, core, t) for t in ("Q5_K", "Q6_K", "Q8_0")},
              "prefill": lambda: prefill_ttft(torch, llm, core),
              "moe": lambda: moe_bench(torch, core),
              "config0": lambda: config0_bench(torch, core), "decode7b": lambda: decode_7b(torch, llm),
              "ggml": lambda: {t: ggml_bench(torch, core, t) for t in ("Q6_K", "Q8_0")}}[a.only]
        out = {a.only: fn()}
        copy_bytes = copy_calibration(torch)
        out.update({"copy_bytes_read": copy_bytes, "copy_bytes_written": copy_bytes})
        print(json.dumps(out), flush=True)
        return
    if a.decode_only:
        m = llm.CausalLM.from_weights(synth.decoder_weights(5, **synth.QWEN2_05B), lmax=max(256, 64 + a.steps + 8))
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
    m_graph_tokens = m.graph_tokens
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
                               "kernel (captured graphs of %d steps, replayed)" % m_graph_tokens,
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
        mf = llm.CausalLM.from_weights(w, lmax=256)
        res["decode_full_128"] = decode_full(torch, mf, ids)
        del mf
        torch.cuda.empty_cache()
        res["config0_gemv_fp16"] = config0_bench(torch, core)
        res["gemv_large"] = gemv_large(torch, core)
        res["q4k_gemv_llama3_8b_up"] = q4k_bench(torch, core)
        res["q6k_gemv_llama3_8b_up"] = ggml_bench(torch, core, "Q6_K")
        res["q8_0_gemv_llama3_8b_up"] = ggml_bench(torch, core, "Q8_0")
        res["q4k_gemm_llama3_8b_up"] = ggml_gemm_bench(torch, core, "Q4_K")
        for t in ("Q5_K", "Q6_K", "Q8_0"):
            res["%s_gemm_llama3_8b_up" % t.lower()] = ggml_gemm_bench(torch, core, t)
        res["prefill64_ttft_llama3_8b_q4_k_m"] = prefill_ttft(torch, llm, core)
        res["gptq_gemm_act_order_4096"] = gemm_bench(torch, core)
        res["gptq_gemm_int8_per_channel_4096"] = gemm_int8_bench(torch, core)
        res["moe_qwen3_t256"] = moe_bench(torch, core)
        res["decode_qwen25_7b_shape"] = decode_7b(torch, llm)
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline(a.cpu_seconds)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
