"""GPU parity: GPTQ dequant / quantizer (bit-exact) and GEMV (tolerance) against the oracle."""
import os

import numpy as np
import pytest

from oracle import gptq
from webpytorch_amd import synth

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _close(got, ref, rtol=1e-2, atol=1e-3):
    """Output parity bar (fp32 accumulate): |got - ref| <= atol + rtol * |ref| elementwise."""
    got = np.asarray(got, np.float64); ref = np.asarray(ref, np.float64)
    bad = np.abs(got - ref) > atol + rtol * np.abs(ref)
    assert not bad.any(), "max err %.3g at %s" % (np.abs(got - ref).max(), np.argwhere(bad)[:3])


def _rel(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / (np.abs(ref).max() + 1e-30))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("sdt", ["f16", "f32"])
@pytest.mark.parametrize("zoff", [0.0, 1.0])
@pytest.mark.parametrize("act", [False, True])
def test_dequant_bit_exact(gpu, bits, sdt, zoff, act):
    import torch
    from webpytorch_amd import core
    L = synth.gptq_layer(21, 512, 264, 128, bits, act_order=act)
    sc = L["scales"] if sdt == "f16" else (L["scales"].astype(np.float32) * np.float32(1.37))
    g_idx = L["g_idx"] if act else None
    W = core.gptq_dequant(core.to_device(L["qweight"]), core.to_device(L["qzeros"]), core.to_device(sc),
                          512, 264, 128, bits, zoff, None if g_idx is None else core.to_device(g_idx))
    ref = gptq.dequant_closed_form(L["qweight"], L["qzeros"], sc, 128, bits, zoff, g_idx=g_idx)
    torch.cuda.synchronize()
    assert np.array_equal(W.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_quantizer_bit_exact_with_reference_golden(gpu):
    from webpytorch_amd import core
    d = np.load(os.path.join(GOLDEN, "gptq_quantize.npz"))
    for n in sorted({k.split(".")[0] for k in d.files}):
        gs, bits, oi, K, N = [int(v) for v in d[n + ".meta"]]
        qw, qz, sc, _, _ = core.gptq_quantize(d[n + ".W"], gs, bits, from_out_in=bool(oi))
        assert np.array_equal(qw.cpu().numpy(), d[n + ".qweight"]), n
        assert np.array_equal(qz.cpu().numpy(), d[n + ".qzeros"]), n
        assert np.array_equal(sc.cpu().numpy().view(np.uint32), d[n + ".scales"].view(np.uint32)), n


def test_quantizer_bit_exact_fp16_head_block(gpu):
    # a head block of the tied embedding: (V, H) fp16 rows quantized from the (out, in) layout
    from webpytorch_amd import core
    emb = (np.random.default_rng(3).standard_normal((4096, 896)) * 0.02).astype(np.float16)
    qw, qz, sc, _, _ = core.gptq_quantize(emb, 128, 4, from_out_in=True)
    r = gptq.gptq_quantize(np.ascontiguousarray(emb.astype(np.float32).T), 128, 4)
    assert np.array_equal(qw.cpu().numpy(), r[0]) and np.array_equal(qz.cpu().numpy(), r[1])
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), r[2].view(np.uint32))


# shapes of the reference's own kernel check (examples/gptq_int4_correctness.py:30-31)
REF_SHAPES = [(128, 64, 32, 4), (256, 128, 128, 4), (3584, 512, 128, 4), (512, 1536, 128, 4),
              (128, 24, 32, 4), (256, 64, 32, 8)]


@pytest.mark.parametrize("K,N,gs,bits", REF_SHAPES)
def test_quantized_linear_matches_numpy_dequant(gpu, K, N, gs, bits):
    """Same procedure as the reference's check: quantize a random weight, compare the layer
    with x @ dequant(W) for M in (1, 3, 4, 5, 32), rel err < 1e-4."""
    import torch
    from webpytorch_amd import core
    rng = np.random.default_rng(0)
    W = (rng.standard_normal((K, N)) * 0.1).astype(np.float32)
    qw, qz, sc, _, _ = gptq.gptq_quantize(W, gs, bits)
    ql = core.QuantizedLinear(qw, qz, sc, np.zeros(N, np.float32), K, N, K, N, gs, bits)
    Wd = gptq.dequant_closed_form(qw, qz, sc, gs, bits, 0.0)
    for M in (1, 3, 4, 5, 32):
        x = (rng.standard_normal((M, K)) * 0.5).astype(np.float32)
        got = ql(torch.from_numpy(x)).cpu().numpy()
        ref = gptq.gptq_matmul_np(x, qw, qz, sc, K, N, gs, bits, 0.0)
        assert _rel(got, ref) < 1e-4, (M, _rel(got, ref))
        assert _rel(got, x.astype(np.float64) @ Wd) < 1e-4


def test_config0_gemv_fp16(gpu):
    """GPTQ int4 GEMV at the Qwen2-0.5B gate_proj shape (x fp16 (1, 896) -> y fp16 (1, 4864))."""
    import torch
    from webpytorch_amd import core
    L = synth.gptq_layer(0, 896, 4864, 128, 4)
    x = synth.activations(0, 1, 896, np.float16)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 128, 4)
    y = ql.forward(torch.from_numpy(x), out_dtype=torch.float16)
    assert y.dtype == torch.float16 and tuple(y.shape) == (1, 4864)
    ref = gptq.gptq_matmul_np(x, L["qweight"], L["qzeros"], L["scales"], 896, 4864, 128, 4, 1.0)
    _close(y.float().cpu().numpy(), ref)
    y32 = ql.forward(torch.from_numpy(x), out_dtype=torch.float32).cpu().numpy()
    assert _rel(y32, ref) < 1e-5
    # repeated calls are deterministic (fixed-order reduction)
    assert np.array_equal(y32, ql.forward(torch.from_numpy(x), out_dtype=torch.float32).cpu().numpy())


@pytest.mark.parametrize("M", [1, 4, 7])
def test_act_order_gemv(gpu, M):
    import torch
    from webpytorch_amd import core
    L = synth.gptq_layer(2, 4096, 4096, 128, 4, act_order=True)
    x = synth.activations(2, M, 4096, np.float16)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 128, 4,
                                            g_idx=L["g_idx"])
    got = ql.forward(torch.from_numpy(x), out_dtype=torch.float32).cpu().numpy()
    ref = gptq.linear_forward(x, L, zoff=1.0, g_idx=L["g_idx"])
    _close(got, ref)
    assert _rel(got, ref) < 1e-5
    W = ql.dequantize().cpu().numpy()
    assert np.array_equal(W, gptq.dequant_closed_form(L["qweight"], L["qzeros"], L["scales"], 128, 4, 1.0,
                                                      g_idx=L["g_idx"]))


@pytest.mark.parametrize("K,N,xdt,sdt,zoff,bias", [
    (4096, 11008, np.float16, "f16", 1.0, False),   # a 7B up projection
    (11008, 4096, np.float32, "f16", 1.0, True),    # a 7B down projection (344 steps of K)
    (896, 65536, np.float32, "f32", 0.0, False),    # a tied-head shape
    (2048, 4096, np.float16, "f32", 1.0, True),
])
def test_large_gemv_matrix_core_path(gpu, K, N, xdt, sdt, zoff, bias):
    """One row against a layer of >= 4 MiB of int4 codes: the matrix-core GEMV (exact bf16
    splits of x, fp32 accumulation) against the numpy-fallback oracle, deterministic."""
    import torch
    from webpytorch_amd import core
    L = synth.gptq_layer(40 + K % 7, K, N, 128, 4)
    sc = L["scales"] if sdt == "f16" else L["scales"].astype(np.float32) * np.float32(1.37)
    x = synth.activations(41, 1, K, np.float16).astype(xdt)
    b = (np.random.default_rng(3).standard_normal(N) * 0.1).astype(np.float32) if bias else None
    out = torch.empty((1, N), dtype=torch.float32, device="cuda")
    args = (torch.from_numpy(x).cuda(), core.to_device(L["qweight"]), core.to_device(L["qzeros"]), core.to_device(sc),
            K, N, 128, 4, zoff)
    got = core._gptq_matmul(*args, bias=None if b is None else core.to_device(b), out=out).cpu().numpy()
    ref = gptq.gptq_matmul_np(x.astype(np.float32), L["qweight"], L["qzeros"], sc, K, N, 128, 4, zoff)
    if b is not None:
        ref = ref + b
    _close(got, ref)
    assert _rel(got, ref) < 1e-5
    again = core._gptq_matmul(*args, bias=None if b is None else core.to_device(b), out=out).cpu().numpy()
    assert np.array_equal(got, again)


@pytest.mark.parametrize("mode,K,N,big", [(1, 3584, 4608, False), (1, 896, 9728, False), (2, 18944, 3584, False),
                                         (2, 4864, 896, False), (1, 1024, 512, True), (2, 512, 768, True),
                                         (1, 3584, 37888, False)])
def test_fused_gemv_matrix_core_path(gpu, mode, K, N, big):
    """One row through miq_gptq_gemv_fused on the matrix-core GEMV: RMSNorm (mode 1, the row's
    mean square over all K in every workgroup, x * w staged, partials divided by r) and SwiGLU
    (mode 2, silu(gate) * up staged) against the oracle's RMSNorm / SwiGLU followed by the numpy
    dequant product; Qwen2.5-7B and Qwen2-0.5B projection shapes, an in-place residual (bias =
    out), a row with values near 1e4, and repeat calls bit-identical."""
    import torch
    from webpytorch_amd import _lib, core
    from webpytorch_amd.core import ptr
    L = synth.gptq_layer(50 + K % 11, K, N, 128, 4)
    rng = np.random.default_rng(K + N)
    eps = 1e-6
    if mode == 1:
        x = rng.standard_normal(K).astype(np.float32) * (3e3 if big else 1.0)
        w = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
        xn = (x / np.sqrt(np.mean(x.astype(np.float64) ** 2) + eps)).astype(np.float32) * w
        xin = x
    else:
        g = rng.standard_normal(K).astype(np.float32) * (8.0 if big else 1.0)
        u = rng.standard_normal(K).astype(np.float32)
        xn = (g / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32) * u
        xin = np.concatenate([g, u])
        w = None
    res = (rng.standard_normal(N) * 0.5).astype(np.float32)
    ref = gptq.gptq_matmul_np(xn[None, :], L["qweight"], L["qzeros"], L["scales"], K, N, 128, 4, 1.0)[0] + res
    xd = torch.from_numpy(xin).cuda()
    wd = None if w is None else torch.from_numpy(w).cuda()
    qw, qz, sc = core.to_device(L["qweight"]), core.to_device(L["qzeros"]), core.to_device(L["scales"])
    ws = core.workspace(core.gemv_workspace_bytes(1, K, N, 128, 4, 0))
    outs = []
    for _ in range(2):
        out = torch.from_numpy(res).cuda()
        _lib.call("miq_gptq_gemv_fused", ptr(xd), mode, None if wd is None else ptr(wd), eps, None, ptr(qw), ptr(qz),
                  ptr(sc), core.dtype_code(sc), ptr(out), ptr(out), 1, K, N, 128, 4, 1.0, ptr(ws), ws.numel(), None)
        outs.append(out.cpu().numpy())
    _close(outs[0], ref)
    assert _rel(outs[0], ref) < 1e-5
    assert np.array_equal(outs[0], outs[1])


def test_int8_per_channel_gemv(gpu):
    import torch
    from webpytorch_amd import core
    L = synth.int8_per_channel_layer(3, 4096, 4096)
    x = synth.activations(3, 2, 4096, np.float16)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 4096, 8)
    got = ql.forward(torch.from_numpy(x), out_dtype=torch.float32).cpu().numpy()
    ref = gptq.gptq_matmul_np(x, L["qweight"], L["qzeros"], L["scales"], 4096, 4096, 4096, 8, 1.0)
    _close(got, ref)
    assert _rel(got, ref) < 1e-5


def test_bias_padding_and_leading_dims(gpu):
    import torch
    from webpytorch_amd import core

    class Lin:  # the reference's Linear stores weight as (in, out)
        pass
    lin = Lin()
    rng = np.random.default_rng(5)
    lin.weight = (rng.standard_normal((200, 60)) * 0.1).astype(np.float32)   # K=200, N=60 -> padded
    lin.bias = rng.standard_normal(60).astype(np.float32)
    ql = core.QuantizedLinear.from_linear(lin, group_size=32, bits=4)
    assert (ql.Kp, ql.Np, ql.Kt, ql.Nt) == (224, 64, 200, 60)
    x = rng.standard_normal((2, 3, 200)).astype(np.float32)
    got = ql(torch.from_numpy(x)).cpu().numpy()
    Wp = np.pad(lin.weight, ((0, 24), (0, 4)))
    qw, qz, sc, _, _ = gptq.gptq_quantize(Wp, 32, 4)
    xp = np.pad(x.reshape(6, 200), ((0, 0), (0, 24)))
    ref = gptq.gptq_matmul_np(xp, qw, qz, sc, 224, 64, 32, 4, 0.0)[:, :60] + lin.bias
    assert got.shape == (2, 3, 60)
    assert _rel(got.reshape(6, 60), ref) < 1e-5


def test_errors_are_raised(gpu):
    import torch
    from webpytorch_amd import core
    with pytest.raises(AssertionError):
        core.QuantizedLinear(np.zeros((4, 8), np.int32), np.zeros((1, 1), np.int32), np.ones((1, 8), np.float16),
                             None, 30, 8, 30, 8, 32, 4)
    with pytest.raises(ValueError, match="g_idx"):
        core.act_order_perm(np.zeros(64, np.int32), 32)


def _random_gemv_cases(n=14, seed=2026):
    """Seeded one-row GEMV cases over the shapes the matrix-core planner handles differently:
    K from one group to 64 groups (one to 32 K-slices, every slice capacity), N from one
    packed word to past 16k columns (ragged last tiles), both activation and scale dtypes, both
    zero offsets, with and without bias."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        K = 128 * int(rng.choice([1, 2, 3, 7, 8, 28, 29, 32, 43, 64]))
        N = 8 * int(rng.integers(1, 40) if i % 2 else rng.integers(500, 2200))
        cases.append((i, K, N, bool(rng.integers(2)), str(rng.choice(["f16", "f32"])), float(rng.integers(2)),
                      bool(rng.integers(2))))
    return cases


@pytest.mark.parametrize("case", _random_gemv_cases(), ids=lambda c: "K%d-N%d" % (c[1], c[2]))
def test_gemv_random_shapes(gpu, case):
    """One row through the drop-in GEMV (matrix-core path for gs 128) against the oracle's
    numpy-fallback product, on seeded random shapes, dtypes, zero offsets and biases."""
    import torch
    from webpytorch_amd import core
    i, K, N, xf16, sdt, zoff, bias = case
    L = synth.gptq_layer(300 + i, K, N, 128, 4)
    sc = L["scales"] if sdt == "f16" else L["scales"].astype(np.float32) * np.float32(0.83)
    x = synth.activations(400 + i, 1, K, np.float16 if xf16 else np.float32)
    b = np.linspace(-0.5, 0.5, N).astype(np.float32) if bias else None
    ref = gptq.gptq_matmul_np(x.astype(np.float32), L["qweight"], L["qzeros"], sc, K, N, 128, 4, zoff)
    if b is not None:
        ref = ref + b
    got = core._gptq_matmul(torch.from_numpy(x).cuda(), core.to_device(L["qweight"]), core.to_device(L["qzeros"]),
                            core.to_device(sc), K, N, 128, 4, zoff,
                            bias=None if b is None else core.to_device(b), out_dtype=torch.float32).cpu().numpy()
    _close(got, ref)
    assert _rel(got, ref) < 1e-5
