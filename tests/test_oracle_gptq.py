"""Pins the GPTQ oracle (CPU): golden vectors from the reference, brute force, closed forms."""
import os

import numpy as np
import pytest

from oracle import gptq
from webpytorch_amd import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def brute_dequant(qweight, qzeros, scales, gs, bits, zoff, g_idx=None):
    """Scalar loops over the AutoGPTQ bit layout, independent of the vectorised oracle."""
    per, mask = 32 // bits, (1 << bits) - 1
    qw = np.asarray(qweight).view(np.uint32)
    qz = np.asarray(qzeros).view(np.uint32)
    K, N = qw.shape[0] * per, qw.shape[1]
    W = np.zeros((K, N), np.float64)
    for k in range(K):
        g = k // gs if g_idx is None else int(g_idx[k])
        for n in range(N):
            q = (int(qw[k // per, n]) >> ((k % per) * bits)) & mask
            z = (int(qz[g, n // per]) >> ((n % per) * bits)) & mask
            W[k, n] = float(np.float32(scales[g, n])) * (q - z - zoff)
    return W


@pytest.mark.parametrize("bits,gs,zoff", [(4, 32, 0.0), (4, 64, 1.0), (8, 32, 1.0), (8, 64, 0.0)])
def test_dequant_matches_brute_force(bits, gs, zoff):
    L = synth.gptq_layer(3, 128, 24 if bits == 4 else 16, gs, bits)
    W = gptq.dequant_closed_form(L["qweight"], L["qzeros"], L["scales"], gs, bits, zoff)
    Wb = brute_dequant(L["qweight"], L["qzeros"], L["scales"], gs, bits, zoff)
    assert np.array_equal(W, Wb.astype(np.float32))


@pytest.mark.parametrize("bits,gs,zoff,M", [(4, 32, 0.0, 1), (4, 128, 1.0, 3), (8, 32, 1.0, 5), (8, 128, 0.0, 2)])
def test_matmul_matches_float64_sum(bits, gs, zoff, M):
    K, N = 256, 40
    L = synth.gptq_layer(5, K, N, gs, bits)
    x = synth.activations(5, M, K, np.float32)
    y = gptq.gptq_matmul_np(x, L["qweight"], L["qzeros"], L["scales"], K, N, gs, bits, zoff, block=16)
    ref = x.astype(np.float64) @ brute_dequant(L["qweight"], L["qzeros"], L["scales"], gs, bits, zoff)
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


def test_matmul_unit_rows_select_weight_rows():
    K, N, gs, bits = 128, 16, 32, 4
    L = synth.gptq_layer(6, K, N, gs, bits)
    W = gptq.dequant_closed_form(L["qweight"], L["qzeros"], L["scales"], gs, bits, 1.0)
    eye = np.eye(K, dtype=np.float32)
    y = gptq.gptq_matmul_np(eye, L["qweight"], L["qzeros"], L["scales"], K, N, gs, bits, 1.0)
    assert np.array_equal(y, W)


def test_code_equal_zero_gives_zero():
    # every code equal to its zero point (+offset) -> exactly zero weights
    K, N, gs, bits = 64, 8, 32, 4
    q = np.full((K, N), 5, np.int64)
    zp = np.full((K // gs, N), 6, np.int64)       # stored as zp-1 = 5, read back +1 = 6 ... -> q - 6
    qw, qz, sc, _ = gptq.pack_autogptq(q, np.ones((K // gs, N)), zp, gs, bits)
    W = gptq.dequant_closed_form(qw, qz, sc, gs, bits, zoff=1.0)
    assert np.all(W == -1.0)
    qw, qz, sc, _ = gptq.pack_autogptq(q, np.ones((K // gs, N)), zp - 1, gs, bits)
    assert np.all(gptq.dequant_closed_form(qw, qz, sc, gs, bits, zoff=1.0) == 0.0)


def test_autogptq_pack_roundtrip():
    g = np.random.default_rng(0)
    K, N, gs, bits = 256, 32, 64, 4
    q = g.integers(0, 16, (K, N))
    zp = g.integers(1, 17, (K // gs, N))          # AutoGPTQ zero points in 1..16
    s = np.abs(g.standard_normal((K // gs, N))).astype(np.float16)
    qw, qz, sc, gi = gptq.pack_autogptq(q, s, zp, gs, bits)
    assert np.array_equal(gptq.unpack_along_k(qw, bits), q)
    assert np.array_equal(gptq.unpack_along_n(qz, bits) + 1, zp % 16 + (zp == 16) * 16)
    W = gptq.dequant_closed_form(qw, qz, sc, gs, bits, zoff=1.0)
    assert np.array_equal(W, (s.astype(np.float32)[gi].astype(np.float64) * (q - zp[gi])).astype(np.float32))
    assert np.array_equal(gi, np.arange(K) // gs)


def test_act_order_permutation_equivalence():
    K, N, gs, bits = 512, 24, 128, 4
    L = synth.gptq_layer(9, K, N, gs, bits, act_order=True)
    x = synth.activations(9, 3, K, np.float32)
    W = gptq.dequant_closed_form(L["qweight"], L["qzeros"], L["scales"], gs, bits, 1.0, g_idx=L["g_idx"])
    Wb = brute_dequant(L["qweight"], L["qzeros"], L["scales"], gs, bits, 1.0, g_idx=L["g_idx"])
    assert np.array_equal(W, Wb.astype(np.float32))
    y = gptq.linear_forward(x, L, zoff=1.0, g_idx=L["g_idx"])
    ref = x.astype(np.float64) @ Wb
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()
    # an identity g_idx leaves the layer unchanged
    xp, qp, perm = gptq.act_order_equivalent(x, L["qweight"], np.arange(K) // gs, bits, gs)
    assert np.array_equal(qp, L["qweight"]) and np.array_equal(perm, np.arange(K))


def test_int8_per_channel_mapping():
    K, N = 256, 16
    L = synth.int8_per_channel_layer(2, K, N)
    W = gptq.dequant_closed_form(L["qweight"], L["qzeros"], L["scales"], K, 8, zoff=1.0)
    expect = (L["scales"].astype(np.float32).astype(np.float64) * L["q"]).astype(np.float32)
    assert np.array_equal(W, expect)


def test_quantize_matches_reference_golden():
    d = np.load(os.path.join(GOLDEN, "gptq_quantize.npz"))
    names = sorted({k.split(".")[0] for k in d.files})
    assert len(names) >= 7
    for n in names:
        gs, bits, oi, K, N = [int(v) for v in d[n + ".meta"]]
        kw = {"from_out_in": True, "block": 32} if oi else {}
        qw, qz, sc, K2, N2 = gptq.gptq_quantize(d[n + ".W"], gs, bits, **kw)
        assert (K2, N2) == (K, N)
        assert np.array_equal(qw, d[n + ".qweight"]), n
        assert np.array_equal(qz, d[n + ".qzeros"]), n
        assert np.array_equal(sc.view(np.uint32), d[n + ".scales"].view(np.uint32)), n


@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_invariants(bits):
    g = np.random.default_rng(4)
    W = (g.standard_normal((256, 32)) * 0.1).astype(np.float32)
    qw, qz, sc, K, N = gptq.gptq_quantize(W, 64, bits)
    qmax = (1 << bits) - 1
    q = gptq.unpack_along_k(qw, bits)
    z = gptq.unpack_along_n(qz, bits)
    assert q.min() >= 0 and q.max() <= qmax and z.min() >= 0 and z.max() <= qmax
    Wd = gptq.dequant_closed_form(qw, qz, sc, 64, bits, zoff=0.0)
    gidx = np.arange(K) // 64
    assert np.all(np.abs(W - Wd) <= sc[gidx] * 0.5 * (1 + 1e-5) + 1e-7)


def test_quantize_rejects_bad_dims():
    with pytest.raises(AssertionError):
        gptq.gptq_quantize(np.zeros((100, 8), np.float32), 32, 4)
