"""GPU parity of the decode engine: each decode-step operator against the oracle's building
blocks, and end-to-end greedy token ids against the reference's own CPU decode (fixtures)."""
import math
import os

import numpy as np
import pytest

from oracle import decode
from webpytorch_amd import synth

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
SHAPE_KEYS = ["L", "H", "NH", "NKV", "HD", "I", "V", "gs", "bits"]


def _state(torch, pos):
    from webpytorch_amd import _lib
    st = torch.zeros(_lib.lib().miq_decode_state_words(), dtype=torch.int32, device="cuda")
    st[0] = pos
    return st


def test_rmsnorm_rope_silu_match_oracle(gpu):
    import torch
    from webpytorch_amd import _lib
    from webpytorch_amd.core import ptr
    o = decode.Qwen2Oracle(synth.decoder_weights(1, L=1, H=128, NH=4, NKV=2, HD=64, I=128, V=64, gs=64), lmax=32)
    rng = np.random.default_rng(0)
    T, H = 5, 128
    x = rng.standard_normal((T, H)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    out = torch.empty((T, H), device="cuda")
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()  # held: raw pointers do not keep tensors alive
    _lib.call("miq_rmsnorm", ptr(xd), ptr(wd), ptr(out), T, H, 1e-6, None)
    np.testing.assert_allclose(out.cpu().numpy(), o.rms(x, w), rtol=2e-6, atol=1e-6)
    # rope + kv write at position 7
    NH, NKV, HD, LMAX, pos = 4, 2, 64, 32, 7
    qkv = rng.standard_normal((T, (NH + 2 * NKV) * HD)).astype(np.float32)
    q = torch.empty((T, NH * HD), device="cuda")
    kc = torch.zeros((NKV, LMAX, HD), device="cuda")
    vc = torch.zeros_like(kc)
    qkvd, st = torch.from_numpy(qkv).cuda(), _state(torch, pos)
    ct, stab = o.rope_tables(0, LMAX)
    cos_t = torch.from_numpy(np.ascontiguousarray(ct[:, :HD // 2])).cuda()
    sin_t = torch.from_numpy(np.ascontiguousarray(stab[:, :HD // 2])).cuda()
    _lib.call("miq_rope_kv", ptr(qkvd), ptr(st), ptr(cos_t), ptr(sin_t), ptr(q), ptr(kc), ptr(vc), T, NH, NKV, HD,
              LMAX, None)
    cos, sin = o.rope_tables(pos, T)
    qr = qkv[:, :NH * HD].reshape(T, NH, HD).transpose(1, 0, 2)
    kr = qkv[:, NH * HD:(NH + NKV) * HD].reshape(T, NKV, HD).transpose(1, 0, 2)
    vr = qkv[:, (NH + NKV) * HD:].reshape(T, NKV, HD).transpose(1, 0, 2)
    qref = qr * cos + o.rot(qr) * sin
    kref = kr * cos + o.rot(kr) * sin
    assert np.array_equal(q.cpu().numpy().reshape(T, NH, HD).transpose(1, 0, 2), qref)
    assert np.array_equal(kc.cpu().numpy()[:, pos:pos + T], kref)
    assert np.array_equal(vc.cpu().numpy()[:, pos:pos + T], vr)
    assert not kc.cpu().numpy()[:, :pos].any() and not kc.cpu().numpy()[:, pos + T:].any()
    # silu * mul
    gu = rng.standard_normal((T, 2 * 96)).astype(np.float32)
    act = torch.empty((T, 96), device="cuda")
    gud = torch.from_numpy(gu).cuda()
    _lib.call("miq_silu_mul", ptr(gud), ptr(act), T, 96, None)
    np.testing.assert_allclose(act.cpu().numpy(), o.silu(gu[:, :96]) * gu[:, 96:], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("pos,T", [(0, 1), (9, 1), (0, 6), (20, 4)])
def test_attention_matches_oracle(gpu, pos, T):
    import torch
    from webpytorch_amd import _lib
    from webpytorch_amd.core import ptr
    NH, NKV, HD, LMAX = 14, 2, 64, 64
    o = decode.Qwen2Oracle(synth.decoder_weights(1, L=1, H=128, NH=2, NKV=1, HD=64, I=128, V=64, gs=64), lmax=LMAX)
    rng = np.random.default_rng(pos * 7 + T)
    kc = rng.standard_normal((NKV, LMAX, HD)).astype(np.float32)
    vc = rng.standard_normal((NKV, LMAX, HD)).astype(np.float32)
    q = rng.standard_normal((T, NH, HD)).astype(np.float32)
    out = torch.empty((T, NH * HD), device="cuda")
    scale = 1.0 / math.sqrt(HD)
    qd, kd, vd, st = (torch.from_numpy(q).cuda(), torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda(),
                      _state(torch, pos))
    _lib.call("miq_attention", ptr(qd), ptr(kd), ptr(vd), ptr(st), ptr(out), T, NH, NKV, HD, LMAX, scale, None)
    S = pos + T
    mask = None
    if T > 1:
        mask = np.triu(np.full((T, S), -1e9, np.float32), 1 + (S - T)).reshape(1, T, S)
    ref = o.attend(q.transpose(1, 0, 2), kc[:, :S], vc[:, :S], mask, scale).transpose(1, 0, 2).reshape(T, NH * HD)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("pos,LMAX,NH,NKV,HD", [(0, 64, 14, 2, 64), (5, 64, 14, 2, 64), (37, 64, 14, 2, 64),
                                                (255, 256, 14, 2, 64), (37, 300, 14, 2, 64), (290, 300, 14, 2, 64),
                                                (0, 64, 28, 4, 128), (63, 200, 28, 4, 128), (191, 200, 28, 4, 128),
                                                (1000, 1030, 28, 4, 128), (2, 40, 8, 8, 128), (700, 800, 4, 1, 80)])
def test_attention_decode_fused_rope_kv(gpu, pos, LMAX, NH, NKV, HD):
    """The one-token attention (RoPE + KV write + attention in one launch) against the oracle's
    rope, cache append and attention: head dim 64 with caches of up to 256 positions takes the
    prefetching kernel, head dims 64 and 128 otherwise the row-group kernel (Qwen2.5-7B's 28/4
    heads of 128 among them), other head dims the looping one."""
    import torch
    from webpytorch_amd import _lib
    from webpytorch_amd.core import ptr
    o = decode.Qwen2Oracle(synth.decoder_weights(1, L=1, H=128, NH=2, NKV=1, HD=HD, I=128, V=64, gs=32), lmax=LMAX)
    rng = np.random.default_rng(pos)
    kc = rng.standard_normal((NKV, LMAX, HD)).astype(np.float32)
    vc = rng.standard_normal((NKV, LMAX, HD)).astype(np.float32)
    qkv = rng.standard_normal((1, (NH + 2 * NKV) * HD)).astype(np.float32)
    ct, stab = o.rope_tables(0, LMAX)
    cos_t = torch.from_numpy(np.ascontiguousarray(ct[:, :HD // 2])).cuda()
    sin_t = torch.from_numpy(np.ascontiguousarray(stab[:, :HD // 2])).cuda()
    kd, vd, qd, st = (torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda(), torch.from_numpy(qkv).cuda(),
                      _state(torch, pos))
    out = torch.empty((1, NH * HD), device="cuda")
    scale = 1.0 / math.sqrt(HD)
    _lib.call("miq_attention_decode", ptr(qd), ptr(st), ptr(cos_t), ptr(sin_t), ptr(kd), ptr(vd), ptr(out), NH, NKV, HD,
              LMAX, scale, None)
    cos, sin = o.rope_tables(pos, 1)
    q = qkv[:, :NH * HD].reshape(1, NH, HD).transpose(1, 0, 2)
    k = qkv[:, NH * HD:(NH + NKV) * HD].reshape(1, NKV, HD).transpose(1, 0, 2)
    v = qkv[:, (NH + NKV) * HD:].reshape(1, NKV, HD).transpose(1, 0, 2)
    q = q * cos + o.rot(q) * sin
    k = k * cos + o.rot(k) * sin
    kref, vref = kc.copy(), vc.copy()
    kref[:, pos:pos + 1], vref[:, pos:pos + 1] = k, v
    assert np.array_equal(kd.cpu().numpy(), kref) and np.array_equal(vd.cpu().numpy(), vref)
    ref = o.attend(q, kref[:, :pos + 1], vref[:, :pos + 1], None, scale).transpose(1, 0, 2).reshape(1, NH * HD)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-6)


def test_argmax_first_index_and_state(gpu):
    import torch
    from webpytorch_amd import _lib
    from webpytorch_amd.core import ptr
    V = 151936
    lg = np.random.default_rng(1).standard_normal(V).astype(np.float32)
    lg[[5000, 90000, 151935]] = lg.max() + 1.0  # ties: the first index wins
    st = _state(torch, 10)
    ids = torch.zeros(4, dtype=torch.int32, device="cuda")
    hist = torch.full((8,), -1, dtype=torch.int32, device="cuda")
    d = torch.from_numpy(lg).cuda()
    for step in range(3):
        _lib.call("miq_argmax_advance", ptr(d), V, ptr(ids), ptr(hist), 8, ptr(st), 1, None)
    s = st.cpu().numpy()
    assert int(ids[0]) == 5000 and list(hist.cpu().numpy()[:4]) == [5000, 5000, 5000, -1]
    assert s[0] == 13 and s[1] == 3 and s[2] == 0 and s[3] == 5000


def _engine(g, lmax):
    from webpytorch_amd import llm
    sh = dict(zip(SHAPE_KEYS, [int(v) for v in g["shape"]]))
    w = synth.decoder_weights(int(g["seed"]), **sh)
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    return llm.CausalLM.from_weights(w, lmax=lmax), ids, w


def test_decode_matches_reference_golden_small(gpu):
    """Greedy ids of the reference's own CPU decode (fixture), reduced shape: eager and replayed."""
    g = np.load(os.path.join(GOLDEN, "decode_small.npz"))
    m, ids, _ = _engine(g, int(g["lmax"]))
    want = [int(t) for t in g["tokens"]]
    assert m.generate(ids, int(g["max_new"]), use_graph=False).tokens == want
    m.fused = False  # the unfused one-token path (separate RMSNorm / RoPE / SwiGLU launches)
    assert m.generate(ids, int(g["max_new"]), use_graph=False).tokens == want
    m.fused = True
    assert m.generate(ids, int(g["max_new"]), use_graph=True).tokens == want
    assert m.generate(ids, int(g["max_new"]), use_graph=True).tokens == want  # graph reused


def test_head_requantization_bit_exact(gpu):
    """The device head equals the oracle's block-wise `_gptq_quantize` of the tied embedding."""
    g = np.load(os.path.join(GOLDEN, "decode_small.npz"))
    m, _, w = _engine(g, 32)
    o = decode.Qwen2Oracle(w, lmax=32)
    qw = np.concatenate([b["qweight"] for b in o.head], axis=1)
    qz = np.concatenate([b["qzeros"] for b in o.head], axis=1)
    sc = np.concatenate([b["scales"] for b in o.head], axis=1)
    assert np.array_equal(m.head.qweight.cpu().numpy(), qw)
    assert np.array_equal(m.head.qzeros.cpu().numpy(), qz)
    assert np.array_equal(m.head.scales.cpu().numpy().view(np.uint32), sc.view(np.uint32))


@pytest.mark.skipif(not os.path.exists(os.path.join(GOLDEN, "decode_qwen2_05b.npz")),
                    reason="full-shape fixture not generated")
def test_decode_matches_reference_golden_qwen2_05b(gpu):
    """End-to-end config: Qwen2-0.5B shape, 64-token prompt, 128 greedy tokens, identical ids."""
    g = np.load(os.path.join(GOLDEN, "decode_qwen2_05b.npz"))
    m, ids, _ = _engine(g, int(g["lmax"]))
    res = m.generate(ids, int(g["max_new"]))
    assert res.tokens == [int(t) for t in g["tokens"]]


def _gauss_engine(g, lmax, persistent=None):
    from webpytorch_amd import llm
    sh = dict(zip(["L", "H", "NH", "NKV", "HD", "I", "V", "gs", "bits"], [int(v) for v in g["shape"]]))
    w = synth.decoder_weights(int(g["seed"]), gaussian=True, **sh)
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    return llm.CausalLM.from_weights(w, lmax=lmax, persistent=persistent), ids


def test_decode_matches_reference_golden_gaussian_small(gpu):
    """Gaussian-quantized weights (varied tokens, every step's top-1/top-2 gap recorded in the
    fixture): the reference's greedy ids, persistent step and launch sequence, eager and
    graph-replayed."""
    g = np.load(os.path.join(GOLDEN, "decode_gauss_small.npz"))
    want = [int(t) for t in g["tokens"]]
    assert len(set(want)) >= 16 and float(g["margins"].min()) > 1e-3
    for persistent in (True, False):
        m, ids = _gauss_engine(g, int(g["lmax"]), persistent)
        assert (m.pws is not None) == persistent
        assert m.generate(ids, int(g["max_new"]), use_graph=False).tokens == want
        assert m.generate(ids, int(g["max_new"])).tokens == want


@pytest.mark.skipif(not os.path.exists(os.path.join(GOLDEN, "decode_gauss_qwen2_05b.npz")),
                    reason="full-shape Gaussian fixture not generated")
def test_decode_matches_reference_golden_gaussian_qwen2_05b(gpu):
    """End-to-end config with varied tokens: Qwen2-0.5B shape, Gaussian-quantized int4 weights,
    64-token prompt, 128 greedy ids identical to the reference's CPU decode, for the persistent
    step and the launch sequence (graph-replayed). The fixture records each step's top-1/top-2
    logit gap; the smallest is far above the engines' logit error (~1e-6 relative)."""
    g = np.load(os.path.join(GOLDEN, "decode_gauss_qwen2_05b.npz"))
    want = [int(t) for t in g["tokens"]]
    assert len(want) == 128 and len(set(want)) >= 30 and float(g["margins"].min()) > 1e-3
    for persistent in (True, False):
        m, ids = _gauss_engine(g, int(g["lmax"]), persistent)
        assert (m.pws is not None) == persistent
        assert m.generate(ids, int(g["max_new"])).tokens == want


def test_decode_moe_qknorm_matches_reference_golden(gpu):
    """Sparse-MoE layers (router GEMV, device routing, grouped expert GEMMs) and per-head q/k
    RMSNorm inside the engine: the reference's greedy ids (its `CausalLM` CPU decode with the
    same layer dicts), eager fused, eager unfused (prefill-style launches per token) and
    graph-replayed with the routing live."""
    from webpytorch_amd import llm
    g = np.load(os.path.join(GOLDEN, "decode_moe_qknorm_small.npz"))
    sh = dict(zip(["L", "H", "NH", "NKV", "HD", "I", "V", "gs", "bits"], [int(v) for v in g["shape"]]))
    ne, mi, k, qk = [int(v) for v in g["extra"]]
    w = synth.decoder_weights(int(g["seed"]), gaussian=True, n_experts=ne, moe_I=mi, top_k=k, qk_norm=bool(qk), **sh)
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    want = [int(t) for t in g["tokens"]]
    m = llm.CausalLM.from_weights(w, lmax=int(g["lmax"]))
    assert m.pws is None  # the persistent step covers dense layers only
    n = int(g["max_new"])
    assert m.generate(ids, n, use_graph=False).tokens == want
    m.fused = False
    assert m.generate(ids, n, use_graph=False).tokens == want
    m.fused = True
    assert m.generate(ids, n).tokens == want
    assert m.generate(ids, n).tokens == want  # the captured graph again, routing re-run per replay


def test_head_rmsnorm_vs_oracle(gpu):
    import torch
    from webpytorch_amd import _lib, core
    T, NH, NKV, HD = 5, 6, 2, 64
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((T, (NH + 2 * NKV) * HD)) * 3).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    qd, kd = torch.from_numpy(qn).cuda(), torch.from_numpy(kn).cuda()  # kept alive across the launch
    _lib.call("miq_head_rmsnorm", core.ptr(xd), core.ptr(qd), core.ptr(kd), T, NH, NKV, HD, 1e-6,
              core.stream_handle())
    got = xd.cpu().numpy()
    o = decode.Qwen2Oracle.__new__(decode.Qwen2Oracle)
    o.eps = 1e-6
    q = o.rms(x[:, :NH * HD].reshape(T, NH, HD), qn).reshape(T, -1)
    k = o.rms(x[:, NH * HD:(NH + NKV) * HD].reshape(T, NKV, HD), kn).reshape(T, -1)
    np.testing.assert_allclose(got[:, :NH * HD], q, rtol=2e-6, atol=1e-6)
    np.testing.assert_allclose(got[:, NH * HD:(NH + NKV) * HD], k, rtol=2e-6, atol=1e-6)
    assert np.array_equal(got[:, (NH + NKV) * HD:], x[:, (NH + NKV) * HD:])


def test_generate_refuses_overlong(gpu):
    g = np.load(os.path.join(GOLDEN, "decode_small.npz"))
    m, ids, _ = _engine(g, 20)
    with pytest.raises(ValueError, match="lmax"):
        m.generate(ids, 10)


def test_decode_varied_tokens_vs_oracle(gpu):
    """A model quantized from Gaussian weights, whose greedy tokens vary (the uniform-code
    models settle on one token): 32 greedy ids identical to the oracle's (itself pinned to the
    reference's CPU decode), eager fused, eager unfused and graph-replayed. Seed chosen so that
    every step's top-1/top-2 logit gap is above 1% of the logits' spread."""
    from webpytorch_amd import llm
    sh = dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, gs=128, bits=4)
    w = synth.decoder_weights(14, gaussian=True, **sh)
    ids = synth.prompt_ids(14, 16, sh["V"])
    want, _ = decode.Qwen2Oracle(w, lmax=64).generate(ids, 32)
    assert len(set(want)) >= 10
    m = llm.CausalLM.from_weights(w, lmax=64)
    assert m.generate(ids, 32, use_graph=False).tokens == want
    m.fused = False
    assert m.generate(ids, 32, use_graph=False).tokens == want
    m.fused = True
    assert m.generate(ids, 32).tokens == want


def test_decode_full_shape_logits_vs_oracle(gpu):
    """End-to-end config weights (Qwen2-0.5B shape, uniform codes): the logits after the 64-token
    prefill and after one decode step against the oracle's, elementwise."""
    import torch
    from webpytorch_amd import llm
    w = synth.decoder_weights(5, **synth.QWEN2_05B)
    ids = synth.prompt_ids(5, 64, synth.QWEN2_05B["V"])
    o = decode.Qwen2Oracle(w, lmax=128)
    cache = [None] * o.L
    n1, l1 = o.forward(list(ids), 0, cache)
    n2, l2 = o.forward([n1], 64, cache)
    m = llm.CausalLM.from_weights(w, lmax=128)
    r = m.generate(ids, 1, use_graph=False)
    g1 = m.buf["logits"][0].cpu().numpy()
    m._step(1)
    torch.cuda.synchronize()
    g2 = m.buf["logits"][0].cpu().numpy()
    assert r.tokens == [n1] and int(m.history[1]) == n2
    for got, ref in ((g1, l1), (g2, l2)):
        bad = np.abs(got - ref) > 1e-3 + 1e-2 * np.abs(ref)
        assert not bad.any(), np.abs(got - ref).max()
        assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-4


def _persistent_pair(sh, seed, lmax, prompt):
    from webpytorch_amd import llm
    w = synth.decoder_weights(seed, gaussian=True, **sh)
    ids = synth.prompt_ids(seed, prompt, sh["V"])
    a = llm.CausalLM.from_weights(w, lmax=lmax, persistent=True)
    b = llm.CausalLM.from_weights(w, lmax=lmax, persistent=False)
    assert a.pws is not None and b.pws is None
    return a, b, ids


@pytest.mark.parametrize("sh,prompt,steps,lmax", [
    (dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, gs=128, bits=4), 16, 24, 64),
    (dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, gs=128, bits=4), 270, 40, 320),
    (dict(synth.QWEN2_05B), 240, 24, 288)])
def test_persistent_step_matches_launch_sequence(gpu, sh, prompt, steps, lmax):
    """The one-launch persistent step against the launch sequence (5 launches per layer) on the
    same model after the same prefill: identical greedy ids and per-step logits within 1e-4
    relative; the second and third cases run past 256 cached positions (the attention's second
    chunk), the third at the full Qwen2-0.5B shape (its role counts, K-slices and GQA grouping)."""
    import torch
    a, b, ids = _persistent_pair(sh, 6 if sh["L"] == 24 else 14, lmax, prompt)
    for m in (a, b):
        m.generate(ids, 1, use_graph=False)
    for step in range(steps):
        for m in (a, b):
            m._step(1)
        torch.cuda.synchronize()
        la, lb = a.buf["logits"][0].cpu().numpy(), b.buf["logits"][0].cpu().numpy()
        assert int(a.history[step + 1]) == int(b.history[step + 1]), step
        np.testing.assert_allclose(la, lb, rtol=1e-4, atol=1e-4 * np.abs(lb).max())
    assert a.persistent_error() == 0
    assert np.array_equal(a.state[:4].cpu().numpy(), b.state[:4].cpu().numpy())
    # the caches the persistent step wrote are the ones the launch sequence wrote (both fp32
    # accumulations, in different orders; the persistent step's int8 matrix-core products hold x
    # in 30-bit fixed point per 64-k step, within 2^-31 of the step's largest value)
    n = prompt + steps
    for ca, cb in ((a.kc, b.kc), (a.vc, b.vc)):
        ga, gb = ca[:, :, :n].cpu().numpy(), cb[:, :, :n].cpu().numpy()
        np.testing.assert_allclose(ga, gb, rtol=1e-4, atol=1e-4 * np.abs(gb).max())


def test_persistent_step_wait_timeout_drains(gpu, monkeypatch):
    """A spin bound of one wall-clock tick makes every waiting workgroup give up: the step ends
    (the grid drains), reports error bit 1 and leaves the decode state alone; after reset() the
    same model decodes the launch sequence's ids."""
    import torch
    sh = dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, gs=128, bits=4)
    a, b, ids = _persistent_pair(sh, 14, 64, 16)
    want = b.generate(ids, 8).tokens
    a.generate(ids, 1, use_graph=False)
    state = a.state.clone()
    monkeypatch.setenv("MIQ_PD_SPIN_TICKS", "1")
    a._step(1)
    torch.cuda.synchronize()
    monkeypatch.delenv("MIQ_PD_SPIN_TICKS")
    assert a.persistent_error() & 1
    assert torch.equal(a.state[:4], state[:4])
    a._step(1)  # the normal bound again: a step after a failed one leaves at entry
    torch.cuda.synchronize()
    assert a.persistent_error() & 1
    assert torch.equal(a.state[:4], state[:4])
    a.reset()
    assert a.persistent_error() == 0
    assert a.generate(ids, 8, use_graph=False).tokens == want and a.fallback_steps == 0


@pytest.mark.parametrize("use_graph", [False, True])
def test_persistent_timeout_falls_back_to_the_launch_sequence(gpu, monkeypatch, use_graph):
    """Steps that time out (a spin bound of one tick, as when another kernel keeps workgroups off
    their CUs) leave the decode state alone, and generate() finishes the sequence with the
    launch sequence: the launch sequence's ids, a RuntimeWarning, every decode step counted."""
    sh = dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, gs=128, bits=4)
    a, b, ids = _persistent_pair(sh, 15, 64, 16)
    want = b.generate(ids, 8).tokens
    monkeypatch.setenv("MIQ_PD_SPIN_TICKS", "1")
    a._graphs.clear()  # captured now, with the one-tick bound
    with pytest.warns(RuntimeWarning, match="launch sequence"):
        got = a.generate(ids, 8, use_graph=use_graph)
    monkeypatch.delenv("MIQ_PD_SPIN_TICKS")
    assert got.tokens == want and a.fallback_steps == 7 and a.persistent_error() == 0
    a._graphs.clear()
    assert a.generate(ids, 8).tokens == want and a.fallback_steps == 0


def test_persistent_step_graph_replay_and_position_guard(gpu):
    """Graph-replayed persistent steps give the eager ids; a step at position LMAX does no work
    and reports error bit 2 (every workgroup leaves at entry), and reset() clears it."""
    import torch
    sh = dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, gs=128, bits=4)
    a, b, ids = _persistent_pair(sh, 14, 64, 16)
    want = b.generate(ids, 20).tokens
    assert a.generate(ids, 20).tokens == want
    assert a.generate(ids, 20, use_graph=False).tokens == want
    a.state[0] = a.lmax
    hist = a.history.clone()
    a._step(1)
    torch.cuda.synchronize()
    assert a.persistent_error() == 2
    assert torch.equal(a.history, hist) and int(a.state[0]) == a.lmax
    a.reset()
    assert a.persistent_error() == 0
    assert a.generate(ids, 20).tokens == want


SMALL = dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, gs=128, bits=4)


@pytest.mark.parametrize("sh,prompt,n", [(SMALL, 16, 12), (dict(synth.QWEN2_05B), 64, 21)])
@pytest.mark.parametrize("persistent", [True, False])
def test_graphs_of_several_steps_match_eager_steps(gpu, sh, prompt, n, persistent):
    """generate() replays graphs of several one-token steps (full graphs of `graph_tokens` and one
    of the remainder): the same ids as the steps run eagerly, bit-identical last logits, KV caches
    and state, for the persistent step and the launch sequence."""
    import torch
    from webpytorch_amd import llm
    seed = 6 if sh["L"] == 24 else 17
    w = synth.decoder_weights(seed, gaussian=True, **sh)
    ids = synth.prompt_ids(seed, prompt, sh["V"])
    a = llm.CausalLM.from_weights(w, lmax=prompt + n + 8, persistent=persistent)
    b = llm.CausalLM.from_weights(w, lmax=prompt + n + 8, persistent=persistent)
    a.graph_tokens = 4 if sh["L"] == 2 else 8
    assert len(a._chunks(n - 1)) == 2  # full graphs and a remainder graph
    ra, rb = a.generate(ids, n), b.generate(ids, n, use_graph=False)
    assert ra.tokens == rb.tokens and sorted(a._graphs) == sorted(t for t, _ in a._chunks(n - 1))
    assert torch.equal(a.state[:4], b.state[:4])
    assert np.array_equal(a.buf["logits"].cpu().numpy().view(np.uint32), b.buf["logits"].cpu().numpy().view(np.uint32))
    m = prompt + n - 1
    for ca, cb in ((a.kc, b.kc), (a.vc, b.vc)):
        assert np.array_equal(ca[:, :, :m].cpu().numpy().view(np.uint32), cb[:, :, :m].cpu().numpy().view(np.uint32))
    assert (a.persistent_error(), b.persistent_error()) == (0, 0)


def test_persistent_graph_stops_at_the_cache_end(gpu):
    """A graph of 8 persistent steps replayed 4 positions before LMAX decodes those 4 tokens (as 4
    eager steps do); the other 4 steps do no work and report error bit 2, the state at LMAX."""
    import torch
    a, b, ids = _persistent_pair(SMALL, 18, 64, 60)
    for m in (a, b):
        m.generate(ids, 1, use_graph=False)
    a.graph(8).replay()
    for _ in range(4):
        b._step(1)
    torch.cuda.synchronize()
    assert a.persistent_error() == 2 and b.persistent_error() == 0
    assert int(a.state[0]) == a.lmax and torch.equal(a.state[:4], b.state[:4])
    assert torch.equal(a.history, b.history)


def test_persistent_trace_matches_untraced_step(gpu):
    """`miq_decode_persistent_trace` computes what `miq_decode_persistent` does (same logits,
    bit for bit, and the same token) and leaves ordered phase marks: for every role workgroup and
    layer, weights issued <= inputs received <= result published, and the kernel's exit after its
    entry; `pd_trace.summarize` reads them."""
    import io
    import torch
    from webpytorch_amd import llm, pd_trace
    sh = dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, gs=128, bits=4)
    w = synth.decoder_weights(16, gaussian=True, **sh)
    ids = synth.prompt_ids(16, 20, sh["V"])
    a = llm.CausalLM.from_weights(w, lmax=64, persistent=True)
    b = llm.CausalLM.from_weights(w, lmax=64, persistent=True)
    for m in (a, b):
        m.generate(ids, 1, use_graph=False)
    t, _ = pd_trace.trace_steps(a, 1)
    b._step(1)
    torch.cuda.synchronize()
    assert np.array_equal(a.buf["logits"].cpu().numpy(), b.buf["logits"].cpu().numpy())
    assert torch.equal(a.state[:4], b.state[:4]) and a.persistent_error() == 0
    roles = pd_trace.role_ranges(a, t)
    for r in roles.values():
        assert len(r) > 0
        for l in range(a.L):
            assert np.all(t[r, l, 0] > 0) and np.all(t[r, l, 0] <= t[r, l, 1]) and np.all(t[r, l, 1] <= t[r, l, 2])
    assert np.all(t[:, a.L + 1, 1] >= t[:, a.L + 1, 0]) and np.all(t[:, a.L, 1] > 0)
    res = pd_trace.summarize(a, t, out=io.StringIO())
    assert set(res["hops"]) == {"qkv->attn", "attn->ored", "ored->gu", "gu->down", "down->qkv"}
