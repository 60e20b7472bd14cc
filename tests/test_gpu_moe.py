"""GPU parity: sparse-MoE MLP (device routing, grouped expert GEMMs, combine) against the
reference's own output on a small instance, against the oracle at the Qwen3-MoE shape, and
under graph capture with the routing live."""
import os

import numpy as np
import pytest

from oracle import moe
from webpytorch_amd import synth

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _check(got, ref, rel):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    bad = np.abs(got - ref) > 1e-3 + 1e-2 * np.abs(ref)
    assert not bad.any(), "max err %.3g at %s" % (np.abs(got - ref).max(), np.argwhere(bad)[:3])
    r = np.abs(got - ref).max() / (np.abs(ref).max() + 1e-30)
    assert r < rel, r


def _layer(w, logits_t):
    return {"moe": {"gate": lambda x: logits_t, "experts": w["experts"], "top_k": w["top_k"],
                    "norm_topk_prob": True, "shared": None}}


def _route_arrays(route, T, k):
    r = route.cpu().numpy().view(np.int32)
    e = r[:T * k].reshape(T, k)
    wts = r[T * k:2 * T * k].view(np.float32).reshape(T, k)
    return e, wts


def test_moe_matches_reference_golden(gpu):
    """The reference's `moe_mlp` output (recorded in the fixture) for T=12, H=128, E=8, I=64,
    top-2, group size 64."""
    import torch
    from webpytorch_amd import core
    g = np.load(os.path.join(GOLDEN, "moe_small.npz"))
    T, H, E, I, k, gs = [int(v) for v in g["dims"]]
    w = synth.moe_workload(int(g["seed"]), T=T, H=H, E=E, I=I, top_k=k, gs=gs)
    lay = _layer(w, torch.from_numpy(w["logits"]).cuda())
    got = core.moe_mlp(None, lay, torch.from_numpy(w["x"]).cuda()).cpu().numpy()
    _check(got, g["y"], rel=1e-5)


@pytest.fixture(scope="module")
def config3():
    w = synth.moe_workload(3)
    ref = moe.moe_mlp_np(w["x"], w["logits"], [moe.gptq_expert(e) for e in w["experts"]], 8)
    return w, ref


def test_config3_qwen3_moe(gpu, config3):
    """Qwen3-MoE-shaped block: T=256, hidden 2048, 128 experts (768 intermediate), top-8."""
    import torch
    from webpytorch_amd import core
    w, ref = config3
    lay = _layer(w, torch.from_numpy(w["logits"]).cuda())
    got = core.moe_mlp(None, lay, torch.from_numpy(w["x"]).cuda()).cpu().numpy()
    _check(got, ref, rel=1e-5)
    # routing: same expert sets, weights equal to the float64 renormalised softmax cast to fp32
    e, wts = _route_arrays(lay["moe"]["_grouped"].last_route, 256, 8)
    idx, wref = moe.route(w["logits"], 8)
    order = np.argsort(idx, axis=1)
    assert np.array_equal(e, np.take_along_axis(idx, order, 1))
    assert np.array_equal(wts, np.take_along_axis(wref, order, 1).astype(np.float32))


def test_moe_single_token_decode(gpu, config3):
    """T = 1 (a decode step) through the same kernels."""
    import torch
    from webpytorch_amd import core
    w, _ = config3
    x1, l1 = w["x"][5:6], w["logits"][5:6]
    ref = moe.moe_mlp_np(x1, l1, [moe.gptq_expert(e) for e in w["experts"]], 8)
    lay = _layer(w, torch.from_numpy(l1).cuda())
    lay["moe"]["_grouped"] = None
    got = core.moe_mlp(None, lay, torch.from_numpy(x1).cuda()).cpu().numpy()
    _check(got, ref, rel=1e-5)


def test_moe_graph_capture_routes_live(gpu):
    """A captured MoE call re-routes on every replay: new logits and tokens written into the
    captured input buffers give the eager result (the reference's captured decode reuses the
    capture-time experts)."""
    import torch
    from webpytorch_amd import core
    w = synth.moe_workload(9, T=4, H=256, E=16, I=128, top_k=4, gs=128)
    ex = core.MoEExperts(w["experts"])
    xb = torch.from_numpy(w["x"]).cuda()
    lb = torch.from_numpy(w["logits"]).cuda()
    ex(xb, lb, 4)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ex(xb, lb, 4)
    rng = np.random.default_rng(0)
    for it in range(4):
        xn = rng.standard_normal(xb.shape).astype(np.float16)
        ln = rng.standard_normal(lb.shape).astype(np.float32)
        xb.copy_(torch.from_numpy(xn))
        lb.copy_(torch.from_numpy(ln))
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        eager = ex(torch.from_numpy(xn).cuda(), torch.from_numpy(ln).cuda(), 4).cpu().numpy()
        assert np.array_equal(got, eager), it
        ref = moe.moe_mlp_np(xn, ln, [moe.gptq_expert(e) for e in w["experts"]], 4)
        _check(got, ref, rel=1e-5)


@pytest.mark.parametrize("T,E,k", [(37, 40, 3), (64, 200, 6), (20, 300, 4), (9, 700, 8), (256, 128, 8),
                                   (3, 1024, 32), (1, 5, 5)])
def test_route_layout(gpu, T, E, k):
    """The whole route buffer against a float64 softmax with top-k by (probability, lowest
    index): picks ascending per token, their renormalised weights, each expert's slots in
    ascending token order, the expert offsets and the 32-row tiles. Row 0 has tied logits."""
    import torch
    from webpytorch_amd import core
    rng = np.random.default_rng(T * 1000 + E)
    lg = rng.standard_normal((T, E)).astype(np.float32)
    lg[0, :E // 2] = lg[0, E // 2]
    nbytes = core.moe_route_bytes(T, E, k)
    route = torch.zeros(nbytes, dtype=torch.uint8, device="cuda")
    lgd = torch.from_numpy(lg).cuda()
    core._lib.call("miq_moe_route", core.ptr(lgd), T, E, k, 1, core.ptr(route), route.numel(),
                   core.stream_handle())
    r = route.cpu().numpy().view(np.int32)
    tk = T * k
    p = moe.softmax_rows(lg)
    order = np.lexsort((np.broadcast_to(np.arange(E), p.shape), -p), axis=1)[:, :k]
    exp_e = np.sort(order, axis=1)
    pw = np.take_along_axis(p, exp_e, 1)
    exp_w = (pw / pw.sum(1, keepdims=True)).astype(np.float32)
    got_e = r[:tk].reshape(T, k)
    got_w = r[tk:2 * tk].view(np.float32).reshape(T, k)
    assert np.array_equal(got_e, exp_e)
    np.testing.assert_allclose(got_w, exp_w, rtol=1e-6, atol=0)
    slot_of, sorted_tok = r[2 * tk:3 * tk], r[3 * tk:4 * tk]
    sorted_w = r[4 * tk:5 * tk].view(np.float32)
    off = r[5 * tk:5 * tk + E + 1]
    cnt = np.bincount(exp_e.ravel(), minlength=E)
    assert np.array_equal(off, np.concatenate([[0], np.cumsum(cnt)]))
    for e in range(E):
        toks = np.nonzero((exp_e == e).any(1))[0]
        assert np.array_equal(sorted_tok[off[e]:off[e + 1]], toks), e
    for i in range(tk):
        s = slot_of[i]
        assert sorted_tok[s] == i // k and sorted_w[s] == got_w.ravel()[i]
    ntiles = r[5 * tk + E + 1]
    t0 = (5 * tk + E + 1 + 1 + 3) & ~3
    tiles = r[t0:t0 + 4 * ntiles].reshape(-1, 4)
    want = [(e, off[e] + r0, min(32, cnt[e] - r0), 0) for e in range(E) for r0 in range(0, cnt[e], 32)]
    assert [tuple(t) for t in tiles] == want


def test_moe_rejects_bad_sizes(gpu):
    from webpytorch_amd import core
    with pytest.raises(NotImplementedError, match="T\\*k"):
        core.moe_route_bytes(1024, 128, 8)
    with pytest.raises(ValueError, match="k="):
        core.moe_route_bytes(4, 8, 9)


# ---- fp32 activations, the shared expert, long batches, non-finite rows ----------------------

@pytest.fixture(scope="module")
def small_moe():
    return synth.moe_workload(12, T=48, H=512, E=16, I=256, top_k=4, gs=128)


@pytest.mark.parametrize("scale", [1.0, 1e-6, 3e5])
def test_moe_fp32_activations(gpu, small_moe, scale):
    """fp32 x (not fp16-representable) against the reference's fp32 multiply: the row-scaled
    hi/lo planes keep fp32 accuracy, also for magnitudes past fp16's range (3e5 * N(0,1)) and
    tiny ones (1e-6, fp16 subnormal)."""
    import torch
    from webpytorch_amd import core
    w = small_moe
    x = (np.random.default_rng(5).standard_normal((48, 512)) * scale).astype(np.float32)
    ref = moe.moe_mlp_np(x, w["logits"], [moe.gptq_expert(e) for e in w["experts"]], 4)
    got = core.MoEExperts(w["experts"])(torch.from_numpy(x).cuda(), torch.from_numpy(w["logits"]).cuda(), 4)
    _check(got.cpu().numpy(), ref, rel=2e-5)


def test_moe_shared_expert_fp32(gpu, small_moe):
    """The shared expert with its sigmoid gate (Qwen-style), fp32 throughout, against the
    oracle's `moe_mlp` tail (`webtorch/lm_engine.py:322-328`); the one-output gate linear is
    quantized from a float weight with padding (from_linear)."""
    import torch
    from webpytorch_amd import core
    w = small_moe
    H = 512
    shared = {n: synth.gptq_layer(13, *(kn if n != "down" else kn[::-1]), 128, 4, name="sh." + n)
              for n, kn in (("gate", (H, 384)), ("up", (H, 384)), ("down", (H, 384)))}

    class Lin:
        pass
    sg = Lin()
    sg.weight = (np.random.default_rng(7).standard_normal((H, 1)) * 0.05).astype(np.float32)
    sg.bias = np.array([0.1], np.float32)
    sgq = core.QuantizedLinear.from_linear(sg, group_size=128, bits=4)
    x = np.random.default_rng(6).standard_normal((48, H)).astype(np.float32)
    lay = {"moe": {"gate": lambda t: torch.from_numpy(w["logits"]).cuda(), "experts": w["experts"], "top_k": 4,
                   "norm_topk_prob": True, "shared": shared, "shared_gate": sgq}}
    got = core.moe_mlp(None, lay, torch.from_numpy(x).cuda()).cpu().numpy()
    from oracle import gptq
    qw, qz, sc, _, _ = gptq.gptq_quantize(np.pad(sg.weight, ((0, 0), (0, 7))), 128, 4)
    gate_fn = moe.gptq_linear({"qweight": qw, "qzeros": qz, "scales": sc, "K": H, "N": 8, "gs": 128, "bits": 4,
                               "bias": np.pad(sg.bias, (0, 7))}, zoff=0.0, n_out=1)
    ref = moe.moe_mlp_np(x, w["logits"], [moe.gptq_expert(e) for e in w["experts"]], 4,
                         shared=moe.gptq_expert(shared), shared_gate=gate_fn)
    _check(got, ref, rel=2e-5)
    # the gate matters: without it the result differs
    lay2 = dict(lay["moe"], shared_gate=None)
    lay2.pop("_shared", None)
    lay2.pop("_grouped", None)
    nog = core.moe_mlp(None, {"moe": lay2}, torch.from_numpy(x).cuda()).cpu().numpy()
    assert np.abs(nog - got).max() > 1e-3


@pytest.mark.parametrize("xdt", [np.float16, np.float32])
def test_moe_experts_with_bias(gpu, small_moe, xdt):
    """Experts whose linears carry fp32 biases (`QuantizedLinear` experts of `_build_layer`,
    `webtorch/llm.py:522-534`): gate / up biases enter before the SwiGLU, the down bias before the
    routing weight, as each expert's forward adds its bias."""
    import torch
    from webpytorch_amd import core
    w = small_moe
    g = np.random.default_rng(21)
    experts, ora = [], []
    for e in w["experts"]:
        d = {n: dict(v, bias=(g.standard_normal(v["N"]) * 0.5).astype(np.float32)) for n, v in e.items()}
        experts.append({n: core.QuantizedLinear.from_autogptq(v["qweight"], v["qzeros"], v["scales"], v["bias"],
                                                              v["gs"], v["bits"]) for n, v in d.items()})
        ora.append(moe.gptq_expert(d))
    x = w["x"].astype(xdt)
    ex = core.MoEExperts(experts)
    assert ex.b["gate"] is not None
    got = ex(torch.from_numpy(x).cuda(), torch.from_numpy(w["logits"]).cuda(), 4).cpu().numpy()
    ref = moe.moe_mlp_np(x.astype(np.float32), w["logits"], ora, 4)
    _check(got, ref, rel=2e-5)
    nob = core.MoEExperts(w["experts"])(torch.from_numpy(x).cuda(), torch.from_numpy(w["logits"]).cuda(), 4)
    assert np.abs(nob.cpu().numpy() - got).max() > 1e-2  # the biases matter


def test_moe_more_picks_than_one_routing_pass(gpu):
    """T * k = 4800 > 4096: routed in blocks of tokens, identical to the oracle."""
    import torch
    from webpytorch_amd import core
    w = synth.moe_workload(14, T=600, H=256, E=16, I=128, top_k=8, gs=128)
    ref = moe.moe_mlp_np(w["x"], w["logits"], [moe.gptq_expert(e) for e in w["experts"]], 8)
    got = core.MoEExperts(w["experts"])(torch.from_numpy(w["x"]).cuda(), torch.from_numpy(w["logits"]).cuda(), 8)
    _check(got.cpu().numpy(), ref, rel=1e-5)


def test_moe_nan_logits_row_routes_to_real_experts(gpu, small_moe):
    """A token whose router logits hold a NaN has NaN probabilities everywhere; it is still sent
    to k real experts (the first ones) with NaN weights, so its output is NaN like the
    reference's and the other tokens' routing and outputs are untouched."""
    import torch
    from webpytorch_amd import core
    w = small_moe
    x = np.random.default_rng(9).standard_normal((48, 512)).astype(np.float32)
    logits = w["logits"].copy()
    logits[5, 2] = np.nan
    ref = moe.moe_mlp_np(x, logits, [moe.gptq_expert(e) for e in w["experts"]], 4)
    got = core.MoEExperts(w["experts"])(torch.from_numpy(x).cuda(), torch.from_numpy(logits).cuda(),
                                        4).cpu().numpy()
    assert np.isnan(ref[5]).all() and np.isnan(got[5]).all()
    keep = np.arange(48) != 5
    _check(got[keep], ref[keep], rel=2e-5)


def test_moe_nan_row_stays_in_its_token(gpu, small_moe):
    import torch
    from webpytorch_amd import core
    w = small_moe
    x = np.random.default_rng(8).standard_normal((48, 512)).astype(np.float32)
    x[3, 100] = np.nan
    ref = moe.moe_mlp_np(x, w["logits"], [moe.gptq_expert(e) for e in w["experts"]], 4)
    got = core.MoEExperts(w["experts"])(torch.from_numpy(x).cuda(), torch.from_numpy(w["logits"]).cuda(),
                                        4).cpu().numpy()
    assert np.isnan(ref[3]).all() and np.isnan(got[3]).all()
    keep = np.arange(48) != 3
    _check(got[keep], ref[keep], rel=2e-5)
