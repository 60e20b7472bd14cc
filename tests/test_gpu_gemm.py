"""GPU parity: the matrix-core GPTQ GEMM (M > 8 rows of fp16 activations) against the oracle,
at the prefill shapes (K = N = 4096, act-order, int8 per-channel) and at ragged ones."""
import numpy as np
import pytest

from oracle import gptq
from webpytorch_amd import synth

pytestmark = pytest.mark.gpu


def _check(got, ref, rel=1e-4):
    """Output parity bar elementwise (|d| <= 1e-3 + 1e-2 |ref|) and a tight max-relative bound."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    bad = np.abs(got - ref) > 1e-3 + 1e-2 * np.abs(ref)
    assert not bad.any(), "max err %.3g at %s" % (np.abs(got - ref).max(), np.argwhere(bad)[:3])
    r = np.abs(got - ref).max() / (np.abs(ref).max() + 1e-30)
    assert r < rel, r


@pytest.mark.parametrize("M", [9, 16, 128, 512])
@pytest.mark.parametrize("act", [False, True])
def test_prefill_gemm_config2(gpu, M, act):
    """GPTQ int4 prefill GEMM, K = N = 4096, gs = 128, with and without act-order."""
    import torch
    from webpytorch_amd import core
    L = synth.gptq_layer(30, 4096, 4096, 128, 4, act_order=act)
    x = synth.activations(30 + M, M, 4096, np.float16)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 128, 4,
                                            g_idx=L["g_idx"] if act else None)
    got = ql.forward(torch.from_numpy(x), out_dtype=torch.float32).cpu().numpy()
    ref = gptq.linear_forward(x, L, zoff=1.0, g_idx=L["g_idx"] if act else None)
    _check(got, ref)
    # fp16 output rounds the same sums once
    y16 = ql.forward(torch.from_numpy(x), out_dtype=torch.float16)
    assert y16.dtype == torch.float16
    assert ql(torch.from_numpy(x)).dtype == torch.float32  # the reference's forward returns fp32
    _check(y16.float().cpu().numpy(), ref, rel=2e-3)


@pytest.mark.parametrize("M", [16, 128, 512])
def test_int8_per_channel_gemm(gpu, M):
    import torch
    from webpytorch_amd import core
    L = synth.int8_per_channel_layer(31, 4096, 4096)
    x = synth.activations(31 + M, M, 4096, np.float16)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 4096, 8)
    got = ql.forward(torch.from_numpy(x), out_dtype=torch.float32).cpu().numpy()
    ref = gptq.gptq_matmul_np(x, L["qweight"], L["qzeros"], L["scales"], 4096, 4096, 4096, 8, 1.0)
    _check(got, ref)
    # the benchmarked call: fp16 out of the same kernel
    got16 = ql.forward(torch.from_numpy(x), out_dtype=torch.float16).float().cpu().numpy()
    _check(got16, ref, rel=2e-3)


@pytest.mark.parametrize("K,N,gs,bits,M", [(256, 264, 32, 4, 20), (384, 136, 64, 4, 33), (512, 520, 128, 8, 17),
                                           (256, 64, 32, 8, 70)])
def test_gemm_ragged_shapes_fp32_scales_bias(gpu, K, N, gs, bits, M):
    """Self-quantized layers (fp32 scales, zero offset 0) with a bias, M not a multiple of 16,
    N not a multiple of 256, small groups."""
    import torch
    from webpytorch_amd import core
    rng = np.random.default_rng(K + N + M)
    W = (rng.standard_normal((K, N)) * 0.1).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    qw, qz, sc, _, _ = gptq.gptq_quantize(W, gs, bits)
    ql = core.QuantizedLinear(qw, qz, sc, b, K, N, K, N, gs, bits)
    x = rng.standard_normal((M, K)).astype(np.float16)
    got = ql.forward(torch.from_numpy(x), out_dtype=torch.float32).cpu().numpy()
    ref = gptq.gptq_matmul_np(x, qw, qz, sc, K, N, gs, bits, 0.0) + b
    _check(got, ref)


def test_gemm_repeated_calls_are_deterministic(gpu):
    """Split-K slices are summed in a fixed order, and the counters re-arm between calls."""
    import torch
    from webpytorch_amd import core
    L = synth.gptq_layer(32, 4096, 1024, 128, 4)
    x = torch.from_numpy(synth.activations(32, 64, 4096, np.float16))
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 128, 4)
    a = ql.forward(x, out_dtype=torch.float32).cpu().numpy()
    for _ in range(3):
        assert np.array_equal(a, ql.forward(x, out_dtype=torch.float32).cpu().numpy())


@pytest.mark.parametrize("K,N,M,sdt,zoff,bias,act", [
    (896, 968, 12, "f32", 0.0, True, False),     # N not a multiple of 64, K of 28 steps
    (4864, 896, 9, "f16", 1.0, False, False),    # two A blocks, ragged last K-slice
    (1024, 200, 16, "f16", 1.0, True, True),     # act-order through the gathered copy
    (4096, 4096, 3, "f16", 1.0, False, False),   # one A block (through the C entry: M <= 8)
    (2048, 1024, 8, "f32", 1.0, True, True),
    (2048, 3080, 16, "f32", 1.0, True, True),    # 16 waves per workgroup over all of K, ragged N
])
def test_few_row_gemm(gpu, K, N, M, sdt, zoff, bias, act):
    """The few-row matrix-core product (M <= 16, gs = 128): exact bf16 halves of the fp16 rows,
    per-group folds, a fixed-point split-K; called through miq_gptq_gemm."""
    import torch
    from webpytorch_amd import core
    L = synth.gptq_layer(60 + M, K, N, 128, 4, act_order=act)
    sc = L["scales"] if sdt == "f16" else L["scales"].astype(np.float32) * np.float32(0.71)
    rng = np.random.default_rng(K + N + M)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    x = synth.activations(61 + M, M, K, np.float16)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], sc, b, 128, 4,
                                            g_idx=L["g_idx"] if act else None)
    ql.zero_offset = zoff
    xd = torch.from_numpy(x).cuda()
    out = torch.empty((M, N), dtype=torch.float32, device="cuda")
    ws = core.workspace(core.gemm_workspace_bytes(M, K, N, 128, 4))
    core._lib.call("miq_gptq_gemm", core.ptr(xd), core.ptr(ql.perm), core.ptr(ql.qweight), core.ptr(ql.qzeros),
                   core.ptr(ql.scales), core.dtype_code(ql.scales), core.ptr(ql.bias), core.ptr(out),
                   core.dtype_code(out), M, K, N, 128, 4, float(zoff), core.ptr(ws), ws.numel(),
                   core.stream_handle())
    got = out.cpu().numpy()
    ref = gptq.linear_forward(x, dict(L, scales=sc), zoff=zoff, g_idx=L["g_idx"] if act else None)
    if b is not None:
        ref = ref + b
    _check(got, ref, rel=1e-5)
    for _ in range(2):  # the fixed-point words re-zero: repeated calls agree bit for bit
        core._lib.call("miq_gptq_gemm", core.ptr(xd), core.ptr(ql.perm), core.ptr(ql.qweight),
                       core.ptr(ql.qzeros), core.ptr(ql.scales), core.dtype_code(ql.scales), core.ptr(ql.bias),
                       core.ptr(out), core.dtype_code(out), M, K, N, 128, 4, float(zoff), core.ptr(ws), ws.numel(),
                       core.stream_handle())
        assert np.array_equal(got, out.cpu().numpy())


@pytest.mark.parametrize("M,act,scale", [(9, False, 1.0), (64, True, 1.0), (200, False, 3e5), (512, True, 1e-4)])
def test_fp32_activation_gemm(gpu, M, act, scale):
    """fp32 activations on the matrix cores (row-scaled fp16 hi/lo rows): the decoder's prefill.
    Against the oracle's fp32 product and a float64 one, including magnitudes beyond fp16's
    range and small ones; NaN in one row stays in that row."""
    import torch
    from webpytorch_amd import core
    K, N = 4096, 1024
    L = synth.gptq_layer(40 + M, K, N, 128, 4, act_order=act)
    x = (np.random.default_rng(M).standard_normal((M, K)) * scale).astype(np.float32)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 128, 4,
                                            g_idx=L["g_idx"] if act else None)
    got = ql(torch.from_numpy(x)).cpu().numpy()
    ref = gptq.linear_forward(x, L, zoff=1.0, g_idx=L["g_idx"] if act else None)
    if scale == 1.0:
        _check(got, ref)
    else:  # the elementwise bar's absolute term is for unit-scale values: compare relative to the scale
        assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5
    W = gptq.dequant_closed_form(L["qweight"], L["qzeros"], L["scales"], 128, 4, 1.0,
                                 g_idx=L["g_idx"] if act else None).astype(np.float64)
    exact = x.astype(np.float64) @ W
    assert np.abs(got - exact).max() / np.abs(exact).max() < 1e-5
    x[1, 7] = np.nan
    got = ql(torch.from_numpy(x)).cpu().numpy()
    assert np.isnan(got[1]).all() and np.isfinite(np.delete(got, 1, 0)).all()
