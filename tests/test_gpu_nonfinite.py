"""GPU parity for NaN, infinities and large magnitudes through every GPTQ product path.

The reference multiplies in numpy fp32 (`_gptq_matmul_np`, `webtorch/_core.py:4046-4072`), so a
NaN activation makes every output NaN, an infinite one makes each output +-Inf (or NaN where the
weight is zero), and large finite activations give large finite outputs. The split-K kernels
here meet their K-slices in fixed-point words; partials those cannot hold take an exact fp32
escape, so the same inputs must give the same non-finite pattern and, for large finite values,
the same numbers to fp32 accuracy.

Paths: one row of fp32 x (matrix-core GEMV, fixed-point split-K), four rows of fp32 x (the
VALU GEMV), four rows of fp16 x (few-row matrix-core GEMM, fixed-point split-K) and 64 rows of
fp16 x (tiled MFMA GEMM, fp32 split-K partials).
"""
import numpy as np
import pytest

from oracle import gptq
from webpytorch_amd import synth

pytestmark = pytest.mark.gpu

K, N, GS = 4096, 1024, 128


def _layer(seed=41):
    return synth.gptq_layer(seed, K, N, GS, 4)


def _run(L, x, scales=None):
    import torch
    from webpytorch_amd import core
    sc = L["scales"] if scales is None else scales
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], sc, None, GS, 4)
    got = ql.forward(torch.from_numpy(x), out_dtype=torch.float32).cpu().numpy()
    ref = gptq.gptq_matmul_np(x.astype(np.float32), L["qweight"], L["qzeros"], np.asarray(sc, np.float32), K, N,
                              GS, 4, 1.0)
    return got, ref


def _same_nonfinite(got, ref):
    """NaN where the reference is NaN; non-finite (the same infinity, or NaN) where it is
    infinite; finite where it is finite."""
    rn, gn = np.isnan(ref), np.isnan(got)
    assert np.array_equal(np.isfinite(got), np.isfinite(ref)), "finite pattern differs"
    assert gn[rn].all(), "NaN lost"
    inf = np.isinf(got)
    assert np.array_equal(got[inf], ref[inf]), "wrong infinity"


PATHS = [(1, np.float32), (4, np.float32), (4, np.float16), (64, np.float16)]


@pytest.mark.parametrize("M,dt", PATHS)
def test_nan_activation_propagates(gpu, M, dt):
    L = _layer()
    x = synth.activations(5, M, K, dt)
    x[:, 1000] = np.nan
    got, ref = _run(L, x)
    assert np.isnan(ref).all()
    _same_nonfinite(got, ref)
    print("M=%d %s: %d NaN of %d" % (M, np.dtype(dt).name, np.isnan(got).sum(), got.size))


@pytest.mark.parametrize("M,dt", PATHS)
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_inf_activation_propagates(gpu, M, dt, sign):
    L = _layer()
    x = synth.activations(6, M, K, dt)
    x[:, 2077] = sign * np.inf
    got, ref = _run(L, x)
    assert not np.isfinite(ref).any()
    _same_nonfinite(got, ref)


@pytest.mark.parametrize("M,dt", PATHS)
def test_nan_in_one_row_stays_in_that_row(gpu, M, dt):
    L = _layer()
    x = synth.activations(7, M, K, dt)
    x[0, 17] = np.nan
    got, ref = _run(L, x)
    _same_nonfinite(got, ref)
    if M > 1:
        err = np.abs(got[1:] - ref[1:]).max() / np.abs(ref[1:]).max()
        assert err < 1e-5, err


@pytest.mark.parametrize("M,dt", [(1, np.float32), (4, np.float32)])
def test_huge_fp32_activations(gpu, M, dt):
    """1e9-scale activations: every K-slice partial is far past the fixed-point range."""
    L = _layer()
    x = (synth.activations(8, M, K, np.float32) * np.float32(1e9)).astype(dt)
    got, ref = _run(L, x)
    assert np.isfinite(got).all()
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err < 1e-5, err


@pytest.mark.parametrize("M,dt", [(1, np.float32), (4, np.float16)])
def test_escape_keeps_the_fixed_point_slices(gpu, M, dt):
    """The first K-slice escapes (group 0 carries a huge scale), the others stay in fixed point;
    the result must hold both: the other slices contribute ~3e3, well above the error bound.
    Checked against the float64 product (the fp32 oracle's own rounding is of the same order)."""
    L = _layer()
    x = synth.activations(9, M, K, np.float32)
    x[:, :GS] *= np.float32(1.0 if dt == np.float32 else 100.0)
    x[:, GS:] *= np.float32(1000.0)
    x = x.astype(dt)
    sc = L["scales"].astype(np.float32)
    sc[0] = 2e5 if dt == np.float32 else 1e4
    got, ref = _run(L, x, scales=sc)
    assert np.isfinite(got).all()
    W = gptq.dequant_closed_form(L["qweight"], L["qzeros"], sc, GS, 4, 1.0).astype(np.float64)
    x64 = x.astype(np.float64)
    exact = x64 @ W
    big = np.abs(exact).max()
    assert big > 4.2e6, big  # past the fixed-point limit (2^22)
    rest = np.abs(x64[:, GS:] @ W[GS:]).max()
    err = np.abs(got.astype(np.float64) - exact).max()
    assert err < 0.1 * rest, (err, rest)  # dropping the fixed-point slices would miss by ~rest
    assert err / big < 1e-5, err / big
    assert np.abs(ref - exact).max() / big < 1e-5
    got2, _ = _run(L, x, scales=sc)  # deterministic: the same bits on a second call
    assert np.array_equal(got, got2)


def test_rows_near_the_fp32_range_through_the_hi_lo_paths(gpu):
    """fp32 rows enter the fp16 matrix cores as hi/lo planes scaled by a power of two chosen per
    row; a finite row whose largest value is ~1e35 (past 2^115) and one of ~1e-30 must come back
    finite and accurate to their own magnitude -- through the GPTQ prefill GEMM (24 fp32 rows),
    the Q4_K prefill GEMM (fp32 rows) and the MoE expert GEMMs (fp32 x)."""
    import torch
    from oracle import moe, q4k
    from webpytorch_amd import core
    M = 24
    mag = np.ones(M, np.float32)
    mag[2], mag[7] = 1e35, 1e-30

    def rows_ok(got, ref):
        assert np.isfinite(got).all()
        for m in range(M):
            assert np.abs(got[m] - ref[m]).max() <= 1e-5 * np.abs(ref[m]).max(), m
    L = _layer()
    x = synth.activations(12, M, K, np.float32) * mag[:, None]
    got, ref = _run(L, x)
    rows_ok(got, ref)
    W = synth.q4k_layer(13, 1024, 256)
    xq = synth.activations(13, M, 1024, np.float32) * mag[:, None]
    got = core.GGMLLinear(W, "Q4_K", 1024, 256)(torch.from_numpy(xq)).cpu().numpy()
    rows_ok(got, q4k.q4k_matmul(xq, W, 1024, 256))
    # MoE: h = silu(g) u squares the scale, so x rows of 1e17 make h rows of ~1e35 (the down
    # projection's row scale) and x rows of 1e-15 make h rows of ~1e-30
    w = synth.moe_workload(14, T=M, H=256, E=8, I=128, top_k=2, gs=128)
    mm = np.ones(M, np.float32)
    mm[2], mm[7] = 1e17, 1e-15
    xm = w["x"].astype(np.float32) * mm[:, None]
    got = core.MoEExperts(w["experts"])(torch.from_numpy(xm).cuda(), torch.from_numpy(w["logits"]).cuda(), 2)
    rows_ok(got.cpu().numpy(), moe.moe_mlp_np(xm, w["logits"], [moe.gptq_expert(e) for e in w["experts"]], 2))
