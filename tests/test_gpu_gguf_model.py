"""GGUF decoders through `CausalLM.from_gguf` (`webtorch/llm.py:856-1129`): small Qwen2-shaped
GGUF files laid out by hand from the format's spec (the writer in test_checkpoint.py), with the
block types mixed per layer as a Q4_K_M file mixes them (Q4_K q/k/gate/up, Q6_K v/down, a Q8_0
token embedding, F32 norms and q/k/v biases) plus an F16 o projection, decoded by the engine and
by the CPU decode oracle over the same weights:
  * weights="native": the engine multiplies the file's blocks; the oracle multiplies their exact
    fp32 dequant (the reference's native layers, `GGMLLinear`);
  * weights="requant": both quantize the dequantized weights to GPTQ int4 (group 128, zero
    offset 0, `_gload_quant`), the tied head included.
Greedy ids must agree at every step whose oracle top-2 logit margin is above the compared
tolerance, and every step's logits must agree to 1e-4 of their range. The sparse-MoE case adds
a router (`ffn_gate_inp`) and stacked experts (`ffn_*_exps`)."""
import numpy as np
import pytest

from oracle import decode, ggml, gptq, q4k
from test_checkpoint import write_gguf
from webpytorch_amd import synth

pytestmark = pytest.mark.gpu

SH = dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048)
TYPES = {"attn_q": "Q4_K", "attn_k": "Q4_K", "attn_v": "Q6_K", "attn_output": "F16",
         "ffn_gate": "Q4_K", "ffn_up": "Q4_K", "ffn_down": "Q6_K"}
IDS = {"F32": 0, "F16": 1, "Q8_0": 8, "Q4_K": 12, "Q6_K": 14}
# fp16 block scales giving |w| ~ 0.02-0.05 (F16: values ~N(0, 0.04^2))
SCALE = {"Q4_K": 1.5e-4, "Q6_K": 3e-5, "Q8_0": 5e-4, "F16": 0.01}


def _dequant(type_name, raw, n):
    if type_name == "Q4_K":
        return q4k.q4k_dequant(np.frombuffer(raw, np.uint8), n)
    return ggml.DEQUANT[type_name][0](np.frombuffer(raw, np.uint8), n)


def _f32(a):
    return np.asarray(a, np.float32).tobytes()


def make_model(path, seed=3, moe=None):
    """Write the GGUF file; return {name: (type, (out, in), raw bytes)} of its matrices and the
    float tensors (norms, biases) as numpy."""
    g = np.random.default_rng(seed)
    L, H, NH, NKV, HD, I, V = (SH[k] for k in ("L", "H", "NH", "NKV", "HD", "I", "V"))
    dims_of = {"attn_q": (NH * HD, H), "attn_k": (NKV * HD, H), "attn_v": (NKV * HD, H), "attn_output": (H, NH * HD),
               "ffn_gate": (I, H), "ffn_up": (I, H), "ffn_down": (H, I)}
    mats, floats, tensors = {}, {}, []

    def mat(name, tname, N, K, s):
        raw = synth.ggml_layer(tname, s, K, N, scale=SCALE[tname]).tobytes()
        mats[name] = (tname, (N, K), raw)
        tensors.append((name, [K, N], IDS[tname], raw))

    def vec(name, v):
        floats[name] = np.asarray(v, np.float32)
        tensors.append((name, [len(v)], 0, _f32(v)))

    mat("token_embd.weight", "Q8_0", V, H, seed * 100 + 1)
    for i in range(L):
        p = "blk.%d." % i
        vec(p + "attn_norm.weight", 1.0 + 0.1 * g.standard_normal(H))
        vec(p + "ffn_norm.weight", 1.0 + 0.1 * g.standard_normal(H))
        for nm, tname in TYPES.items():
            if moe and nm.startswith("ffn_"):
                continue
            N, K = dims_of[nm]
            mat(p + nm + ".weight", tname, N, K, seed * 100 + 10 * i + len(nm))
        for nm in ("attn_q", "attn_k", "attn_v"):
            vec(p + nm + ".bias", 0.02 * g.standard_normal(dims_of[nm][0]))
        if moe:
            E, mI = moe["E"], moe["I"]
            mat(p + "ffn_gate_inp.weight", "Q8_0", E, H, seed * 100 + 50 + i)
            for nm, (N, K), tname in (("ffn_gate_exps", (mI, H), "Q4_K"), ("ffn_up_exps", (mI, H), "Q4_K"),
                                      ("ffn_down_exps", (H, mI), "Q6_K")):
                raws = [synth.ggml_layer(tname, seed * 1000 + 97 * i + 7 * e + len(nm), K, N,
                                         scale=SCALE[tname]).tobytes() for e in range(E)]
                raw = b"".join(raws)
                mats[p + nm + ".weight"] = (tname, (E, N, K), raw)
                tensors.append((p + nm + ".weight", [K, N, E], IDS[tname], raw))
    vec("output_norm.weight", 1.0 + 0.1 * g.standard_normal(H))
    kv = [("general.architecture", 8, "qwen2"), ("qwen2.embedding_length", 4, H), ("qwen2.block_count", 4, L),
          ("qwen2.attention.head_count", 4, NH), ("qwen2.attention.head_count_kv", 4, NKV),
          ("qwen2.feed_forward_length", 4, I), ("qwen2.context_length", 4, 4096),
          ("qwen2.attention.layer_norm_rms_epsilon", 6, 1e-6), ("qwen2.rope.freq_base", 6, 1000000.0)]
    if moe:
        kv += [("qwen2.expert_count", 4, moe["E"]), ("qwen2.expert_used_count", 4, moe["k"]),
               ("qwen2.expert_feed_forward_length", 4, moe["I"])]
    write_gguf(str(path), kv, tensors)
    return mats, floats


def oracle_weights(mats, floats, mode, moe=None):
    """Oracle weights over the file's tensors, built the reference's way: every matrix, the MoE
    router and each expert included, as its exact fp32 dequant (native: `_gload_native`,
    `_gexperts`, `webtorch/llm.py:731-783`) or as GPTQ int4 of it (requant: `_gload_quant`)."""
    L, H, NH, NKV, HD, I, V = (SH[k] for k in ("L", "H", "NH", "NKV", "HD", "I", "V"))

    def dense(name):
        tname, shape, raw = mats[name]
        return _dequant(tname, raw, int(np.prod(shape))).reshape(shape)

    def layer(W, bias=None):
        if mode == "native":
            return {"W": W, "bias": bias}
        N, K = W.shape  # `_gload_quant` pads N to the pack width (a 4-expert router: 4 -> 8)
        Np = N + (-N) % 8
        qw, qz, sc, _, _ = gptq.gptq_quantize(np.ascontiguousarray(np.pad(W, ((0, Np - N), (0, 0)))), 128, 4,
                                              from_out_in=True)
        return {"qweight": qw, "qzeros": qz, "scales": sc, "K": K, "N": Np, "Nt": N, "gs": 128, "bits": 4,
                "zoff": 0.0, "bias": bias}


    layers = []
    for i in range(L):
        p = "blk.%d." % i
        lay = {"in_ln": floats[p + "attn_norm.weight"], "post_ln": floats[p + "ffn_norm.weight"]}
        for key, nm in (("q", "attn_q"), ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output")):
            lay[key] = layer(dense(p + nm + ".weight"), floats.get(p + nm + ".bias"))
        if moe:
            st = {k: dense(p + "ffn_%s_exps.weight" % k) for k in ("gate", "up", "down")}
            lay["moe"] = {"router": layer(dense(p + "ffn_gate_inp.weight")), "top_k": moe["k"],
                          "experts": [{k: layer(st[k][e]) for k in st} for e in range(moe["E"])]}
        else:
            for key, nm in (("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down")):
                lay[key] = layer(dense(p + nm + ".weight"))
        layers.append(lay)
    emb = dense("token_embd.weight")
    w = {"layers": layers, "embed": emb, "final_norm": floats["output_norm.weight"],
         "cfg": dict(L=L, H=H, NH=NH, NKV=NKV, HD=HD, V=V, gs=128, bits=4, eps=1e-6, theta=1e6)}
    if mode == "native":
        w["head_W"] = emb
    return w


def _compare(m, ora, ids, steps, tol=1e-4):
    import torch
    want, logs = ora.generate(ids, steps + 1, keep_logits=True)
    m.generate(ids, 1, use_graph=False)
    got = [int(m.history[0])]
    np.testing.assert_allclose(m.buf["logits"][0].cpu().numpy(), logs[0], rtol=tol, atol=tol * np.abs(logs[0]).max())
    for s in range(steps):
        m._step(1)
        torch.cuda.synchronize()
        got.append(int(m.history[s + 1]))
        np.testing.assert_allclose(m.buf["logits"][0].cpu().numpy(), logs[s + 1], rtol=tol,
                                   atol=tol * np.abs(logs[s + 1]).max())
    # greedy ids agree wherever the oracle's choice is not within the tolerance of a tie
    checked = 0
    for s, lg in enumerate(logs):
        top2 = np.sort(lg)[-2:]
        if top2[1] - top2[0] > 10 * tol * np.abs(lg).max():
            assert got[s] == want[s], (s, got, want)
            checked += 1
        else:
            break  # later steps follow different histories after a near-tie
    assert checked >= 4, "too few discriminating steps (%d)" % checked
    return got


@pytest.mark.parametrize("mode", ["native", "requant"])
def test_gguf_decoder_matches_oracle(gpu, tmp_path, mode):
    from webpytorch_amd import llm
    path = tmp_path / "m.gguf"
    mats, floats = make_model(path, seed=4)  # seed 4: no oracle near-tie in the first 11 steps
    m = llm.CausalLM.from_gguf(str(path), lmax=64, weights=mode)
    assert m.native_gguf == (mode == "native") and m.bits == 4
    if mode == "native":
        # v (Q6_K) next to q/k (Q4_K): a column group of q|k concatenated and v; gate|up share
        # Q4_K: one concatenated matrix; the F16 o projection multiplied as stored
        from webpytorch_amd import core
        g = m.layers[0]["qkv"]
        assert isinstance(g, llm._Group) and [p.type_name for p in g.parts] == ["Q4_K", "Q6_K"]
        assert g.parts[0].Nt == (SH["NH"] + SH["NKV"]) * SH["HD"]
        assert isinstance(m.layers[0]["gate_up"], core.GGMLLinear) and m.layers[0]["gate_up"].Nt == 2 * SH["I"]
        assert isinstance(m.head, core.GGMLLinear) and m.head.type_name == "Q8_0"
        assert isinstance(m.layers[0]["o"], core.GGMLLinear) and m.layers[0]["o"].type_name == "F16"
    ora = decode.Qwen2Oracle(oracle_weights(mats, floats, mode), lmax=64)
    ids = synth.prompt_ids(4, 9, SH["V"])
    _compare(m, ora, ids, 10)
    # the captured step replays the same ids
    want = m.generate(ids, 8, use_graph=False).tokens
    assert m.generate(ids, 8, use_graph=True).tokens == want


@pytest.mark.parametrize("mode", ["native", "requant"])
def test_gguf_moe_decoder_matches_oracle(gpu, tmp_path, mode):
    """Native: the Q8_0 router and the Q4_K / Q6_K experts stay in their encoding (the grouped
    GGUF expert GEMV); requant: all quantized to GPTQ int4 (the GPTQ expert GEMMs)."""
    from webpytorch_amd import llm
    moe = dict(E=4, k=2, I=256)
    path = tmp_path / "moe.gguf"
    mats, floats = make_model(path, seed=5, moe=moe)
    m = llm.CausalLM.from_gguf(str(path), lmax=64, weights=mode)
    assert m.has_moe and m.layers[0]["moe"]["experts"].native == (mode == "native")
    ora = decode.Qwen2Oracle(oracle_weights(mats, floats, mode, moe), lmax=64)
    _compare(m, ora, synth.prompt_ids(5, 7, SH["V"]), 8)
    want = m.generate(synth.prompt_ids(5, 7, SH["V"]), 6, use_graph=False).tokens
    assert m.generate(synth.prompt_ids(5, 7, SH["V"]), 6, use_graph=True).tokens == want


def test_gguf_from_pretrained_and_source_bits(gpu, tmp_path):
    from webpytorch_amd import checkpoint, llm
    path = tmp_path / "m.gguf"
    make_model(path)
    g = checkpoint.GGUFFile(str(path))
    assert checkpoint.gguf_source_bits(g) == 4  # Q4_K holds most of the layer weights
    # dtype="int8" sets the width of what is quantized; natively decodable weights stay native
    # unless weights="requant" (`AutoModelForCausalLM._load_raw`, `webtorch/_sdk.py:98-110`)
    m = llm.AutoModelForCausalLM.from_pretrained(str(path), dtype="int8", lmax=64)
    assert m.bits == 8 and m.native_gguf
    m = llm.AutoModelForCausalLM.from_pretrained(str(path), dtype="int8", lmax=64, weights="requant")
    assert m.bits == 8 and not m.native_gguf and m.head.bits == 8
    with pytest.raises(ValueError):
        llm.CausalLM.from_gguf(str(path), weights="fp32")
