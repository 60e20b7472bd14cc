"""GPU parity for the GGUF types beyond the K-quants -- the i-quant grids (IQ2_XXS, IQ2_XS, IQ2_S,
IQ3_XXS, IQ3_S, IQ1_S, IQ1_M), TQ1_0 / TQ2_0, MXFP4 / NVFP4, Q1_0 / Q2_0 and unquantized F32 /
F16 / BF16 matrices -- and for GGUF sparse-MoE experts kept in their block encoding:
  * device dequant bit for bit against the reference's own `ggufload.dequant` output
    (tests/golden/ggml_ext.npz) and against the oracle on random blocks;
  * the GEMV (`ggml_matmul` / `GGMLLinear`) against the oracle's exact dequant times x;
  * `moe_mlp` over native experts (`miq_moe_ggml_gemv`) against the oracle MoE with the experts'
    exact dequant (the reference's native `_gexperts` layers)."""
import os

import numpy as np
import pytest

from webpytorch_amd import synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ggml_ext.npz")
EXT = ["IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S", "IQ1_S", "IQ1_M", "TQ1_0", "TQ2_0", "MXFP4", "NVFP4",
       "Q1_0", "Q2_0"]
DENSE = ["F32", "F16", "BF16"]


def _rel(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / (np.abs(ref).max() + 1e-30))


def _cases():
    z = np.load(GOLDEN)
    n = len({k.split(".")[0] for k in z.files})
    return [(str(z["c%02d.type" % i]), z["c%02d.raw" % i], z["c%02d.y" % i]) for i in range(n)]


@pytest.mark.parametrize("case", range(len(_cases())))
def test_dequant_matches_reference_fixture(gpu, case):
    import torch
    from webpytorch_amd import core
    name, raw, want = _cases()[case]
    vals = core._NATIVE_TYPES[name][0]
    got = core.ggml_dequant(torch.from_numpy(raw.copy()).cuda(), name, want.size // vals).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name


@pytest.mark.parametrize("name", EXT)
def test_dequant_random_blocks_bit_exact(gpu, name):
    """Random code, index, sign and sub-scale bytes; fp16 scale fields of mixed sign and magnitude
    (subnormals included, finite); MXFP4 / NVFP4 scale bytes fully random."""
    import torch
    from oracle import ggml
    from webpytorch_amd import core
    f, vals, nbytes = ggml.DEQUANT[name]
    g = np.random.default_rng(vals * 1000 + nbytes)
    nb = 1531
    raw = g.integers(0, 256, (nb, nbytes), dtype=np.uint8)
    for off in ggml.F16_FIELDS[name]:
        h = (g.standard_normal(nb) * np.exp2(g.integers(-26, 6, nb))).astype(np.float16)
        raw[:, off:off + 2] = h.view(np.uint8).reshape(nb, 2)
    if name == "IQ1_M":  # d's fp16 bits sit in the top nibbles of the four scale words
        d = (g.standard_normal(nb) * np.exp2(g.integers(-20, 6, nb))).astype(np.float16).view(np.uint16).astype(np.int64)
        for k in range(4):
            raw[:, 49 + 2 * k] = (raw[:, 49 + 2 * k] & 0x0F) | (((d >> (4 * k)) & 15) << 4).astype(np.uint8)
    got = core.ggml_dequant(torch.from_numpy(raw.reshape(-1)).cuda(), name, nb).cpu().numpy()
    ref = f(raw.reshape(-1), nb * vals)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name", EXT + DENSE)
@pytest.mark.parametrize("M", [1, 3])
def test_gemv_matches_oracle(gpu, name, M):
    """A 4096 -> 2048 layer in each type, one and three activation rows (fp16), fp32 out."""
    import torch
    from oracle import ggml
    from webpytorch_amd import core
    K, N = 4096, 2048
    W = synth.ggml_layer(name, 3, K, N)
    x = synth.activations(3, M, K, np.float16)
    got = core.GGMLLinear(W, name, K, N)(torch.from_numpy(x)).cpu().numpy()
    ref = ggml.ggml_matmul(x, W, name, K, N)
    assert got.shape == (M, N) and _rel(got, ref) < 1e-5
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))


@pytest.mark.parametrize("name", EXT + DENSE)
def test_ragged_rows_bias_dtypes(gpu, name):
    """Few blocks per row at odd byte offsets, a ragged row count, bias, fp32 and fp16
    activations, fp16 output, and GGMLLinear.dequantize bit-exact."""
    import torch
    from oracle import ggml
    from webpytorch_amd import core
    vals = ggml.DEQUANT[name][1]
    K = 3 * vals if vals >= 128 else (7 * vals if vals > 1 else 100)  # F16 K = 100: rows 8-byte aligned
    N = 37
    W = synth.ggml_layer(name, K + N, K, N)
    b = np.linspace(-1, 1, N).astype(np.float32)
    lin = core.GGMLLinear(W, name, K, N, bias=b)
    for xdt in (np.float32, np.float16):
        x = synth.activations(K, 2, K, xdt)
        ref = ggml.ggml_matmul(x, W, name, K, N) + b
        got = lin(torch.from_numpy(x)).cpu().numpy()
        assert _rel(got, ref) < 1e-5
        got16 = lin.forward(torch.from_numpy(x), out_dtype=torch.float16).cpu().numpy()
        assert got16.dtype == np.float16
        assert np.all(np.abs(got16.astype(np.float32) - ref) <= 1e-3 + 1e-2 * np.abs(ref))
    deq = lin.dequantize().cpu().numpy()
    ref = ggml.DEQUANT[name][0](W.reshape(-1), N * K).reshape(N, K)
    assert np.array_equal(deq.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("name", ["IQ2_XS", "IQ3_S", "IQ1_M", "TQ1_0", "MXFP4", "NVFP4", "F16", "BF16"])
def test_prefill_rows(gpu, name):
    import torch
    from oracle import ggml
    from webpytorch_amd import core
    K, N = 2048, 96
    W = synth.ggml_layer(name, 11, K, N)
    x = synth.activations(11, 24, K, np.float32)
    got = core.GGMLLinear(W, name, K, N)(torch.from_numpy(x)).cpu().numpy()
    ref = ggml.ggml_matmul(x, W, name, K, N)
    assert _rel(got, ref) < 1e-5
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))


def test_native_supported_covers_the_reference_table():
    """Every type of the reference's native table (`webtorch/_core.py:3609-3637`)."""
    from webpytorch_amd import core
    names = ["F32", "F16", "BF16", "TQ1_0", "TQ2_0", "MXFP4", "NVFP4", "Q1_0", "Q2_0", "Q4_0", "Q4_1", "Q5_0", "Q5_1",
             "Q8_0", "IQ4_NL", "IQ4_XS", "Q4_K", "Q5_K", "Q6_K", "Q3_K", "Q2_K", "IQ2_XXS", "IQ2_XS", "IQ2_S",
             "IQ3_XXS", "IQ3_S", "IQ1_S", "IQ1_M"]
    assert all(core.ggml_native_supported(n) for n in names) and len(names) == 28
    assert not core.ggml_native_supported("Q8_K")


# ---- sparse-MoE experts kept in their GGUF encoding -------------------------------------------

def _native_experts(types, E, H, I, seed):
    """E experts of GGMLLinear gate/up (H -> I) and down (I -> H) in the given block types, with
    the oracle's callables over their exact fp32 dequant."""
    from oracle import ggml, q4k
    from webpytorch_amd import core
    deq = {"Q4_K": lambda raw, n: q4k.q4k_dequant(raw, n)}
    exps, ora = [], []
    for e in range(E):
        d, o = {}, {}
        for name, (K, N) in (("gate", (H, I)), ("up", (H, I)), ("down", (I, H))):
            t = types[name]
            W = synth.ggml_layer(t, seed * 1000 + 17 * e + len(name), K, N, scale=0.004)
            d[name] = core.GGMLLinear(W, t, K, N)
            Wd = deq.get(t, ggml.DEQUANT.get(t, (None,))[0])(W.reshape(-1), N * K).reshape(N, K)
            o[name] = (lambda Wd_: (lambda x: np.asarray(x, np.float32) @ Wd_.T))(Wd)
        exps.append(d)
        ora.append(o)
    return exps, ora


@pytest.mark.parametrize("types,T,xdt", [
    ({"gate": "Q4_K", "up": "Q4_K", "down": "Q6_K"}, 1, np.float32),   # a Q4_K_M file's experts, decode
    ({"gate": "Q4_K", "up": "Q4_K", "down": "Q6_K"}, 19, np.float16),  # prefill rows
    ({"gate": "IQ2_XS", "up": "IQ2_XS", "down": "IQ3_S"}, 7, np.float32),
    ({"gate": "MXFP4", "up": "MXFP4", "down": "MXFP4"}, 5, np.float32),
    ({"gate": "Q8_0", "up": "Q5_K", "down": "Q8_0"}, 6, np.float32),   # gate and up of different types
])
def test_moe_native_experts_match_oracle(gpu, types, T, xdt):
    import torch
    from oracle import moe as omoe
    from webpytorch_amd import core
    E, H, I, k = 8, 512, 256, 3
    exps, ora = _native_experts(types, E, H, I, seed=T)
    g = np.random.default_rng(T)
    x = g.standard_normal((T, H)).astype(xdt)
    logits = g.standard_normal((T, E)).astype(np.float32)
    ex = core.MoEExperts(exps)
    assert ex.native and ex.fused_gate_up == (types["gate"] == types["up"])
    got = ex(torch.from_numpy(x).cuda(), torch.from_numpy(logits).cuda(), k).cpu().numpy()
    ref = omoe.moe_mlp_np(x.astype(np.float32), logits, ora, k)
    assert _rel(got, ref) < 1e-5
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))


def test_moe_native_experts_through_moe_mlp_and_capture(gpu):
    """`moe_mlp` with a native router and native experts; the same call captured in a graph and
    replayed with new router logits routes live."""
    import torch
    from oracle import moe as omoe
    from webpytorch_amd import core
    E, H, I, k, T = 6, 256, 256, 2, 4
    types = {"gate": "Q4_K", "up": "Q4_K", "down": "Q4_K"}
    exps, ora = _native_experts(types, E, H, I, seed=4)
    g = np.random.default_rng(4)
    x = torch.from_numpy(g.standard_normal((T, H)).astype(np.float32)).cuda()
    lg = torch.from_numpy(g.standard_normal((T, E)).astype(np.float32)).cuda()
    lay = {"moe": {"gate": lambda t: lg, "experts": exps, "top_k": k, "norm_topk_prob": True, "shared": None}}
    out = core.moe_mlp(None, lay, x)
    ref = omoe.moe_mlp_np(x.cpu().numpy(), lg.cpu().numpy(), ora, k)
    assert _rel(out.cpu().numpy(), ref) < 1e-5
    ex = lay["moe"]["_grouped"]
    res = torch.empty((T, H), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ex._block(x, lg, k, True, res)
    for seed in (5, 6):
        lg.copy_(torch.from_numpy(np.random.default_rng(seed).standard_normal((T, E)).astype(np.float32)))
        graph.replay()
        torch.cuda.synchronize()
        ref = omoe.moe_mlp_np(x.cpu().numpy(), lg.cpu().numpy(), ora, k)
        assert _rel(res.cpu().numpy(), ref) < 1e-5
