"""Write golden vectors by running the REFERENCE's own numpy path (run in the build container
only; `/root/reference` never travels with the repository).

Only functions that no closed form pins are recorded here:
  * `_gptq_quantize` bit patterns (round-half-even ties, constant groups, int8,
    from_out_in) -- `webtorch/_core.py:3782-3824`
  * `lm_engine.moe_mlp` output on a small seeded instance -- `webtorch/lm_engine.py:294-333`
  * `CausalLM.generate` greedy token ids on the CPU growing-cache path, at a reduced shape and
    at the full Qwen2-0.5B shape, for uniform-code and Gaussian-quantized AutoGPTQ models, with
    each step's top-1/top-2 logit gap -- `webtorch/llm.py:1716-1787`
  * the same for a plain fp16 model quantized on load to int4 and int8 (`from_fp16(quantize=)`,
    `webtorch/llm.py:1211-1257, 835-853`), also at sizes the quantizer pads (K and N,
    `webtorch/llm.py:843-849`) with a sparse-MoE layer
  * `ggufload.dequant` of random blocks of the GGUF types beyond the K-quants (the i-quant
    grids, TQ1_0/TQ2_0, MXFP4/NVFP4, Q1_0/Q2_0, F32/F16/BF16), whose bit layouts no closed
    form fixes -- `webtorch/ggufload.py:133-505`

Inputs are regenerated from seeds by `webpytorch_amd.synth`; the fixtures hold the seeds,
the shapes and the reference's outputs. Usage: python tests/golden/make_golden.py [--full] [--only name,...]
"""
import argparse
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.abspath(os.path.join(HERE, "..", "..")))
REF = "/root/reference"

from webpytorch_amd import synth  # noqa: E402


def import_reference():
    # The reference falls back to numpy when its browser array backend cannot be imported
    # (`webtorch/_core.py:11-17`); that fallback is the CPU path recorded here.
    sys.path.insert(0, REF)
    from webtorch import _core as wt
    from webtorch import lm_engine, llm
    assert wt.xp is np and not wt.GPU, "reference did not take its numpy fallback"
    return wt, lm_engine, llm


# ggml type ids of the types the ggml_ext fixture covers
EXT_TYPES = {"IQ2_XXS": 16, "IQ2_XS": 17, "IQ3_XXS": 18, "IQ1_S": 19, "IQ3_S": 21, "IQ2_S": 22, "IQ1_M": 29,
             "BF16": 30, "TQ1_0": 34, "TQ2_0": 35, "MXFP4": 39, "NVFP4": 40, "Q1_0": 41, "Q2_0": 42,
             "F32": 0, "F16": 1}


def ext_cases():
    """(type, raw bytes, n values): seeded random blocks with finite scale fields, plus blocks
    with the scale encodings' edge patterns (MXFP4 exponents 0, 1, 2, 254; NVFP4 scale bytes 0,
    0x7F, 0x80, 0xFF, 0x07, 0x08)."""
    cases = []
    for name in EXT_TYPES:
        vals = synth.GGML_BLOCKS[name][0] if name in synth.GGML_BLOCKS else 1
        K = max(256, 4 * vals) if vals > 1 else 64
        raw = synth.ggml_layer(name, 77, K, 6 if vals > 1 else 3, scale=0.01)
        cases.append((name, raw.tobytes(), raw.size // (synth.GGML_BLOCKS[name][1] if vals > 1 else
                                                         synth.DENSE_TYPES[name]) * vals))
    g = np.random.default_rng(78)
    mx = g.integers(0, 256, (4, 17), dtype=np.uint8)
    mx[:, 0] = [0, 1, 2, 254]
    cases.append(("MXFP4", mx.tobytes(), 4 * 32))
    nv = g.integers(0, 256, (2, 36), dtype=np.uint8)
    nv[:, 0:4] = [[0, 0x7F, 0x80, 0xFF], [0x07, 0x08, 0x3F, 0x79]]
    cases.append(("NVFP4", nv.tobytes(), 2 * 64))
    return cases


def make_ggml_ext(out):
    sys.path.insert(0, REF)
    from webtorch import ggufload
    d = {}
    for i, (name, raw, n) in enumerate(ext_cases()):
        y = ggufload.dequant(EXT_TYPES[name], raw, n)
        d["c%02d.type" % i] = np.array(name)
        d["c%02d.raw" % i] = np.frombuffer(raw, np.uint8)
        d["c%02d.y" % i] = np.asarray(y, np.float32)
    np.savez_compressed(out, **d)


def quantize_cases():
    g = np.random.default_rng(1234)
    cases = []
    # plain random weights, int4 gs=32
    cases.append(("rand_b4_g32", (g.standard_normal((256, 64)) * 0.1).astype(np.float32), 32, 4, False))
    # values on a coarse grid: many w/scale land exactly on .5 (half-even ties)
    grid = (g.integers(-8, 8, (256, 64)) * 0.125).astype(np.float32)
    cases.append(("ties_b4_g32", grid, 32, 4, False))
    # constant groups (scale 0 -> 1e-8), mixed with a normal column block
    const = np.repeat(g.standard_normal((1, 64)).astype(np.float32), 128, 0)
    const[:, 32:] = (g.standard_normal((128, 32)) * 0.05).astype(np.float32)
    cases.append(("const_b4_g64", const, 64, 4, False))
    # all-zero weight
    cases.append(("zeros_b4_g32", np.zeros((64, 16), np.float32), 32, 4, False))
    # int8 groups of 128
    cases.append(("rand_b8_g128", (g.standard_normal((256, 64)) * 0.1).astype(np.float32), 128, 8, False))
    # (out, in) layout with a column block smaller than N
    cases.append(("outin_b4_g128", (g.standard_normal((96, 256)) * 0.02).astype(np.float32), 128, 4, True))
    # fp16-origin head rows (the tied-embedding head requantization)
    emb = (g.standard_normal((40, 128)) * 0.02).astype(np.float16)
    cases.append(("head_b4_g128", np.ascontiguousarray(emb.astype(np.float32).T), 128, 4, False))
    return cases


def make_quantize(wt, out):
    d = {}
    for name, W, gs, bits, oi in quantize_cases():
        kw = {"from_out_in": True, "block": 32} if oi else {}
        qw, qz, sc, K, N = wt._gptq_quantize(W, gs, bits, **kw)
        d[name + ".W"] = W
        d[name + ".meta"] = np.array([gs, bits, int(oi), K, N], np.int64)
        d[name + ".qweight"] = qw
        d[name + ".qzeros"] = qz
        d[name + ".scales"] = sc
    np.savez_compressed(out, **d)


class _Lm:
    def __init__(self, H):
        self.H = H


def make_moe(wt, lm_engine, out, seed=7, T=12, H=128, E=8, I=64, top_k=2, gs=64):
    w = synth.moe_workload(seed, T=T, H=H, E=E, I=I, top_k=top_k, gs=gs)
    experts = []
    for ex in w["experts"]:
        experts.append({k: wt.QuantizedLinear.from_autogptq(v["qweight"], v["qzeros"],
                                                             v["scales"], None, gs, 4)
                        for k, v in ex.items()})
    logits = w["logits"]
    moe = {"gate": lambda x: wt.Tensor(logits), "top_k": top_k, "norm_topk_prob": True,
           "experts": experts, "shared": None}
    x = wt.Tensor(w["x"].astype(np.float32))
    y = lm_engine.moe_mlp(_Lm(H), {"moe": moe}, x).numpy()
    np.savez_compressed(out, seed=seed, dims=np.array([T, H, E, I, top_k, gs]), y=y)


class _Tok:
    eot = -1
    eos_ids = []

    def decode(self, ids):
        return ""


def build_reference_lm(wt, llm, wts, lmax):
    c = wts["cfg"]
    m = llm.CausalLM("")
    m._apply_cfg({"hidden_size": c["H"], "num_hidden_layers": c["L"],
                  "num_attention_heads": c["NH"], "num_key_value_heads": c["NKV"],
                  "head_dim": c["HD"], "vocab_size": c["V"], "rms_norm_eps": 1e-6,
                  "rope_theta": 1e6, "tie_word_embeddings": True})
    m.gs, m.bits, m.lmax = c["gs"], c["bits"], lmax
    m.tok = _Tok()
    m.gen_defaults = {}
    m._gpu = False
    m.embed = wts["embed"]
    m.head = m._quantize_head(m.embed)

    def ql(d):
        b = d.get("bias")
        return wt.QuantizedLinear.from_autogptq(d["qweight"], d["qzeros"], d["scales"],
                                                None if b is None else b.astype(np.float32),
                                                d["gs"], d["bits"])
    m.layers = []
    for lay in wts["layers"]:
        d = {"in_ln": wt.Tensor(lay["in_ln"].astype(np.float32)),
             "post_ln": wt.Tensor(lay["post_ln"].astype(np.float32)),
             "q": ql(lay["q"]), "k": ql(lay["k"]), "v": ql(lay["v"]), "o": ql(lay["o"]),
             "qn": None if lay.get("qn") is None else wt.Tensor(lay["qn"].astype(np.float32)),
             "kn": None if lay.get("kn") is None else wt.Tensor(lay["kn"].astype(np.float32))}
        if lay.get("moe"):  # the layer dict `_build_layer` makes for a sparse layer (`llm.py:522-534`)
            mo = lay["moe"]
            d["moe"] = {"gate": ql(mo["router"]), "top_k": mo["top_k"], "norm_topk": True,
                        "experts": [{k: ql(e[k]) for k in ("gate", "up", "down")} for e in mo["experts"]]}
        else:
            d.update({"gate": ql(lay["gate"]), "up": ql(lay["up"]), "down": ql(lay["down"])})
        m.layers.append(d)
    m.final_norm = wt.Tensor(wts["final_norm"].astype(np.float32))
    m._init_state()
    return m


def _generate_with_margins(m, ids, max_new):
    """The reference's greedy generate, recording each step's top-1 minus top-2 logit and the
    logits' spread (max - min) as `_pick` sees them."""
    margins, spreads = [], []
    pick = m._pick

    def recording_pick(logits):
        lg = np.asarray(logits, np.float32)
        top = np.partition(lg, -2)[-2:]
        margins.append(float(top[1] - top[0]))
        spreads.append(float(lg.max() - lg.min()))
        return pick(logits)
    m._pick = recording_pick
    t0 = time.time()
    res = m.generate(ids=[int(i) for i in ids], max_new=max_new)
    return res.tokens, np.asarray(margins, np.float32), np.asarray(spreads, np.float32), time.time() - t0


SHAPE_KEYS = ("L", "H", "NH", "NKV", "HD", "I", "V", "gs", "bits")


def make_decode(wt, llm, out, seed, shape, prompt_len, max_new, lmax, gaussian=False, **extra):
    wts = synth.decoder_weights(seed, gaussian=gaussian, **shape, **extra)
    ids = synth.prompt_ids(seed, prompt_len, shape["V"])
    m = build_reference_lm(wt, llm, wts, lmax)
    toks, margins, spreads, dt = _generate_with_margins(m, ids, max_new)
    print("%s: %d tokens (%d distinct) in %.1fs, min margin %.3g" % (os.path.basename(out), len(toks),
                                                                     len(set(toks)), dt, margins.min()))
    np.savez_compressed(out, seed=seed, prompt_len=prompt_len, max_new=max_new, lmax=lmax,
                        gaussian=int(gaussian), shape=np.array([shape[k] for k in SHAPE_KEYS]),
                        tokens=np.asarray(toks, np.int64), margins=margins, spreads=spreads,
                        extra=np.array([int(extra.get(k, 0)) for k in ("n_experts", "moe_I", "top_k", "qk_norm")]))


def build_reference_fp16q(wt, llm, model, bits, lmax, gs=128):
    """The reference's `CausalLM.from_fp16(quantize=bits)` composition (`webtorch/llm.py:1211-1257`,
    `_gquant` 835-853, `_quantize_head` 594-602) on the tensors of `synth.fp16_decoder`: every
    (out, in) projection read as fp32 from its fp16 bytes and quantized on load."""
    c, t = model["config"], model["tensors"]
    m = llm.CausalLM("")
    m._apply_cfg(dict(c))
    m.gs, m.bits, m._qbits, m.lmax = gs, bits, bits, lmax
    m.tok = _Tok()
    m.gen_defaults = {}
    m._gpu = False
    m.embed = t["model.embed_tokens.weight"]
    m.head = m._quantize_head(m.embed)

    def lin(prefix):
        b = t.get(prefix + ".bias")
        return m._mklin(t[prefix + ".weight"].astype(np.float32), None if b is None else b.astype(np.float32))
    m.layers = []
    for i in range(c["num_hidden_layers"]):
        p = "model.layers.%d." % i
        lay = {"in_ln": wt.Tensor(t[p + "input_layernorm.weight"].astype(np.float32)),
               "post_ln": wt.Tensor(t[p + "post_attention_layernorm.weight"].astype(np.float32)),
               "q": lin(p + "self_attn.q_proj"), "k": lin(p + "self_attn.k_proj"),
               "v": lin(p + "self_attn.v_proj"), "o": lin(p + "self_attn.o_proj"), "qn": None, "kn": None}
        if m._is_moe_layer(i):  # the sparse block `_build_layer` makes (`llm.py:522-534`)
            lay["moe"] = {"gate": lin(p + "mlp.gate"), "top_k": m.top_k, "norm_topk": m.norm_topk,
                          "experts": [{n: lin(p + "mlp.experts.%d.%s_proj" % (e, n)) for n in ("gate", "up", "down")}
                                      for e in range(m.n_experts)]}
        else:
            lay.update({"gate": lin(p + "mlp.gate_proj"), "up": lin(p + "mlp.up_proj"),
                        "down": lin(p + "mlp.down_proj")})
        m.layers.append(lay)
    m.final_norm = wt.Tensor(t["model.norm.weight"].astype(np.float32))
    m._init_state()
    return m


def make_fp16q(wt, llm, out, seed, shape, prompt_len, max_new, lmax, **moe):
    """Greedy ids of a plain fp16 model loaded with quantize-on-load to int4 and to int8."""
    model = synth.fp16_decoder(seed, **shape, **moe)
    ids = synth.prompt_ids(seed, prompt_len, shape["V"])
    d = {}
    for bits in (4, 8):
        m = build_reference_fp16q(wt, llm, model, bits, lmax)
        toks, margins, spreads, dt = _generate_with_margins(m, ids, max_new)
        print("%s int%d: %d tokens (%d distinct) in %.1fs, min margin %.3g" % (
            os.path.basename(out), bits, len(toks), len(set(toks)), dt, margins.min()))
        d["tokens_int%d" % bits] = np.asarray(toks, np.int64)
        d["margins_int%d" % bits] = margins
    np.savez_compressed(out, seed=seed, prompt_len=prompt_len, max_new=max_new, lmax=lmax,
                        shape=np.array([shape[k] for k in ("L", "H", "NH", "NKV", "HD", "I", "V")]),
                        moe=np.array([moe.get("n_experts", 0), moe.get("moe_I", 0), moe.get("top_k", 0)]),
                        mlp_only=np.array(sorted(moe.get("mlp_only", ())), np.int64), **d)


SMALL = dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, gs=128, bits=4)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--full", action="store_true", help="also the full Qwen2-0.5B-shaped decode")
    ap.add_argument("--full-only", action="store_true", help="only the full Qwen2-0.5B-shaped decode")
    ap.add_argument("--only", default="", help="comma-separated fixture names to (re)write")
    a = ap.parse_args()
    wt, lm_engine, llm = import_reference()
    only = set(filter(None, a.only.split(",")))

    def want(name, default):
        return name in only if only else default
    if want("ggml_ext", not a.full_only):
        make_ggml_ext(os.path.join(HERE, "ggml_ext.npz"))
    if want("gptq_quantize", not a.full_only):
        make_quantize(wt, os.path.join(HERE, "gptq_quantize.npz"))
    if want("moe_small", not a.full_only):
        make_moe(wt, lm_engine, os.path.join(HERE, "moe_small.npz"))
    if want("decode_small", not a.full_only):
        make_decode(wt, llm, os.path.join(HERE, "decode_small.npz"), 11, SMALL, 16, 24, 64)
    # Gaussian-quantized models: varied greedy tokens; seed 14 (reduced shape) and seed 6 (full
    # shape) were chosen for their smallest per-step top-1/top-2 logit gap (recorded in the file)
    if want("decode_gauss_small", not a.full_only):
        make_decode(wt, llm, os.path.join(HERE, "decode_gauss_small.npz"), 14, SMALL, 16, 32, 64, gaussian=True)
    # Qwen3-MoE-style layers: sparse MoE MLPs (8 experts of 128, top-2) and per-head q/k RMSNorm;
    # seed 33 chosen for its varied ids and smallest top-1/top-2 gap
    if want("decode_moe_qknorm_small", not a.full_only):
        make_decode(wt, llm, os.path.join(HERE, "decode_moe_qknorm_small.npz"), 33, SMALL, 16, 32, 64, gaussian=True,
                    n_experts=8, moe_I=128, top_k=2, qk_norm=1)
    if want("decode_fp16q_small", not a.full_only):
        make_fp16q(wt, llm, os.path.join(HERE, "decode_fp16q_small.npz"), 21, SMALL, 16, 32, 64)
    # sizes the quantizer pads: intermediate 200 (the down projection's K to 256) and a 60-expert
    # router (N to 64 at int4) in a model whose layer 0 is dense and layer 1 sparse
    if want("decode_fp16q_pad_moe_small", not a.full_only):
        make_fp16q(wt, llm, os.path.join(HERE, "decode_fp16q_pad_moe_small.npz"), 23,
                   dict(SMALL, I=200), 16, 24, 64, n_experts=60, moe_I=128, top_k=4, mlp_only=(0,))
    if want("decode_qwen2_05b", a.full or a.full_only):
        make_decode(wt, llm, os.path.join(HERE, "decode_qwen2_05b.npz"), 5, dict(synth.QWEN2_05B),
                    64, 128, 256)
    if want("decode_gauss_qwen2_05b", a.full or a.full_only):
        make_decode(wt, llm, os.path.join(HERE, "decode_gauss_qwen2_05b.npz"), 6, dict(synth.QWEN2_05B),
                    64, 128, 256, gaussian=True)


if __name__ == "__main__":
    main()
