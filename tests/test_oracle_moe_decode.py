"""Pins the MoE and decode oracles (CPU): reference golden vectors and closed forms."""
import os

import numpy as np
import pytest

from oracle import decode, moe
from webpytorch_amd import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def test_moe_matches_reference_golden():
    g = np.load(os.path.join(GOLDEN, "moe_small.npz"))
    T, H, E, I, k, gs = [int(v) for v in g["dims"]]
    w = synth.moe_workload(int(g["seed"]), T=T, H=H, E=E, I=I, top_k=k, gs=gs)
    y = moe.moe_mlp_np(w["x"], w["logits"], [moe.gptq_expert(e) for e in w["experts"]], k)
    assert np.array_equal(y, g["y"])


def test_moe_closed_form_identity_experts():
    # gate = up = down = identity -> each token gets sum_j w_j * silu(x) * x = silu(x) * x
    T, H, E, k = 5, 8, 4, 2
    g = np.random.default_rng(0)
    x = g.standard_normal((T, H)).astype(np.float32)
    logits = g.standard_normal((T, E))
    ident = {"gate": lambda t: t, "up": lambda t: t, "down": lambda t: t}
    y = moe.moe_mlp_np(x, logits, [ident] * E, k)
    ref = x * (1 / (1 + np.exp(-x))) * x
    assert np.allclose(y, ref, rtol=1e-6, atol=1e-6)
    # routing picks the k largest logits and the weights sum to 1
    idx, wts = moe.route(logits, k)
    assert np.array_equal(np.sort(idx, 1), np.sort(np.argsort(-logits, 1)[:, :k], 1))
    assert np.allclose(wts.sum(1), 1.0)
    # expert e scales by (e+1): output = sum_j w_j (e_j+1)^3 silu-free product
    sc = [{"gate": (lambda t, a=e + 1.0: t * a), "up": (lambda t: t), "down": (lambda t: t)} for e in range(E)]
    y2 = moe.moe_mlp_np(x, logits, sc, k)
    p = np.exp(logits - logits.max(1, keepdims=True)); p /= p.sum(1, keepdims=True)
    ref2 = np.zeros_like(x, dtype=np.float64)
    for t in range(T):
        top = np.argsort(-logits[t])[:k]
        ww = p[t, top] / p[t, top].sum()
        for e, wj in zip(top, ww):
            a = x[t] * (e + 1.0)
            ref2[t] += wj * (a / (1 + np.exp(-a))) * x[t]
    assert np.allclose(y2, ref2, rtol=1e-5, atol=1e-6)


def test_decode_matches_reference_golden_small():
    g = np.load(os.path.join(GOLDEN, "decode_small.npz"))
    sh = dict(zip(["L", "H", "NH", "NKV", "HD", "I", "V", "gs", "bits"], [int(v) for v in g["shape"]]))
    o = decode.Qwen2Oracle(synth.decoder_weights(int(g["seed"]), **sh), lmax=int(g["lmax"]))
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    toks, _ = o.generate(ids, int(g["max_new"]))
    assert toks == [int(t) for t in g["tokens"]]


def _tiny():
    sh = dict(L=1, H=128, NH=2, NKV=1, HD=64, I=128, V=64, gs=64, bits=4)
    return decode.Qwen2Oracle(synth.decoder_weights(2, **sh), lmax=32)


def test_rope_is_a_rotation():
    o = _tiny()
    x = np.random.default_rng(0).standard_normal((2, 3, 64)).astype(np.float32)
    cos, sin = o.rope_tables(5, 3)
    y = x * cos + o.rot(x) * sin
    # pairs (i, i + 32) rotate by angle pos * theta^(-2i/64): norms kept, angle as closed form
    for t in range(3):
        ang = (5 + t) * (1e6 ** (-np.arange(0, 64, 2) / 64.0))
        a, b = x[:, t, :32], x[:, t, 32:]
        ya = a * np.cos(ang) - b * np.sin(ang)
        yb = b * np.cos(ang) + a * np.sin(ang)
        assert np.allclose(y[:, t, :32], ya, atol=1e-5) and np.allclose(y[:, t, 32:], yb, atol=1e-5)


def test_rmsnorm_and_softmax_closed_form():
    o = _tiny()
    x = np.random.default_rng(1).standard_normal((3, 128)).astype(np.float32)
    w = np.linspace(0.5, 1.5, 128).astype(np.float32)
    y = o.rms(x, w)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * w
    assert np.allclose(y, ref, rtol=1e-5)
    s = o.softmax(x)
    assert np.allclose(s.sum(-1), 1, atol=1e-6) and np.argmax(s[0]) == np.argmax(x[0])


def test_prefill_equals_stepwise_decode():
    # the causal mask makes a T-token prefill equal to feeding the tokens one at a time
    o = _tiny()
    ids = [3, 9, 27, 1]
    c1 = [None] * o.L
    _, l1 = o.forward(ids, 0, c1)
    c2 = [None] * o.L
    for p, t in enumerate(ids):
        _, l2 = o.forward([t], p, c2)
    assert np.allclose(l1, l2, rtol=1e-4, atol=1e-5)


def test_decode_matches_reference_golden_gaussian_small():
    """Gaussian-quantized weights: varied greedy ids of the reference's CPU decode (fixture)."""
    g = np.load(os.path.join(GOLDEN, "decode_gauss_small.npz"))
    assert int(g["gaussian"]) == 1
    sh = dict(zip(["L", "H", "NH", "NKV", "HD", "I", "V", "gs", "bits"], [int(v) for v in g["shape"]]))
    o = decode.Qwen2Oracle(synth.decoder_weights(int(g["seed"]), gaussian=True, **sh), lmax=int(g["lmax"]))
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    toks, logs = o.generate(ids, int(g["max_new"]), keep_logits=True)
    want = [int(t) for t in g["tokens"]]
    assert toks == want and len(set(want)) >= 16
    # the oracle's logits carry the reference's top-1/top-2 gaps
    gaps = [float(np.diff(np.partition(lg, -2)[-2:])[0]) for lg in logs]
    np.testing.assert_allclose(gaps, g["margins"], rtol=1e-3, atol=1e-5)


@pytest.mark.parametrize("bits", [4, 8])
def test_fp16_quantize_on_load_matches_reference_golden(bits):
    """A plain fp16 model quantized on load (`from_fp16(quantize=bits)`: gs 128, zero offset 0,
    fp32 scales; int8 is group-128 asymmetric): the reference's greedy ids."""
    g = np.load(os.path.join(GOLDEN, "decode_fp16q_small.npz"))
    sh = dict(zip(["L", "H", "NH", "NKV", "HD", "I", "V"], [int(v) for v in g["shape"]]))
    model = synth.fp16_decoder(int(g["seed"]), **sh)
    o = decode.Qwen2Oracle(decode.fp16q_weights(model["tensors"], model["config"], bits), lmax=int(g["lmax"]))
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    toks, _ = o.generate(ids, int(g["max_new"]))
    want = [int(t) for t in g["tokens_int%d" % bits]]
    assert toks == want and len(set(want)) >= 16


def pad_moe_model():
    """The fixture model whose sizes the quantizer pads: intermediate 200 in the dense layer 0
    (the down projection's K to 256) and a 60-expert router in the sparse layer 1 (N to 64 at
    int4, unpadded at int8)."""
    g = np.load(os.path.join(GOLDEN, "decode_fp16q_pad_moe_small.npz"))
    sh = dict(zip(["L", "H", "NH", "NKV", "HD", "I", "V"], [int(v) for v in g["shape"]]))
    ne, mi, k = [int(v) for v in g["moe"]]
    model = synth.fp16_decoder(int(g["seed"]), **sh, n_experts=ne, moe_I=mi, top_k=k,
                               mlp_only=tuple(int(v) for v in g["mlp_only"]))
    return g, sh, model


@pytest.mark.parametrize("bits", [4, 8])
def test_fp16_quantize_on_load_pads_like_the_reference(bits):
    """Quantize-on-load pads K to the group multiple and N to the pack width and slices the
    outputs back (`_gquant`, `webtorch/llm.py:843-849`; `QuantizedLinear.forward`,
    `webtorch/_core.py:4446-4456`): the reference's greedy ids for such a model."""
    g, sh, model = pad_moe_model()
    w = decode.fp16q_weights(model["tensors"], model["config"], bits)
    assert w["layers"][0]["down"]["K"] == 256 and w["layers"][0]["down"]["Kt"] == 200
    assert w["layers"][1]["moe"]["router"]["N"] == (64 if bits == 4 else 60)
    o = decode.Qwen2Oracle(w, lmax=int(g["lmax"]))
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    toks, _ = o.generate(ids, int(g["max_new"]))
    assert toks == [int(t) for t in g["tokens_int%d" % bits]]


def _moe_fixture():
    g = np.load(os.path.join(GOLDEN, "decode_moe_qknorm_small.npz"))
    sh = dict(zip(["L", "H", "NH", "NKV", "HD", "I", "V", "gs", "bits"], [int(v) for v in g["shape"]]))
    ne, mi, k, qk = [int(v) for v in g["extra"]]
    w = synth.decoder_weights(int(g["seed"]), gaussian=True, n_experts=ne, moe_I=mi, top_k=k, qk_norm=bool(qk), **sh)
    return g, sh, w


def test_decode_moe_qknorm_matches_reference_golden():
    """Sparse-MoE layers (router, 8 experts, top-2) with per-head q/k RMSNorm: the oracle's
    greedy ids and per-step logit gaps equal those of the reference's `CausalLM` CPU decode."""
    g, sh, w = _moe_fixture()
    o = decode.Qwen2Oracle(w, lmax=int(g["lmax"]))
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    toks, logs = o.generate(ids, int(g["max_new"]), keep_logits=True)
    assert toks == [int(t) for t in g["tokens"]] and len(set(toks)) >= 16
    gaps = [float(np.diff(np.partition(lg, -2)[-2:])[0]) for lg in logs]
    np.testing.assert_allclose(gaps, g["margins"], rtol=1e-3, atol=1e-5)
    # the QK-norm is what the reference applied: without it the ids differ
    for lay in w["layers"]:
        lay.pop("qn"), lay.pop("kn")
    assert decode.Qwen2Oracle(w, lmax=int(g["lmax"])).generate(ids, int(g["max_new"]))[0] != toks
