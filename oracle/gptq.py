"""GPTQ oracle (test infrastructure only; see `oracle/__init__.py`).

Pins:
  * `gptq_matmul_np` -- brute-force float64 sums on small shapes, the AutoGPTQ closed form
    (`dequant_closed_form`), special cases (q = z + zoff gives 0; unit activations select a
    row), and golden vectors written by the reference itself (`tests/golden/`).
  * `gptq_quantize` -- golden vectors from the reference's `_gptq_quantize` (ties, constant
    groups, int8), plus the invariants |w - s*(q - z)| <= s/2 and 0 <= q, z <= qmax.
  * `dequant_closed_form` with `g_idx` (act-order) -- the row-permutation equivalence onto
    `gptq_matmul_np` and brute force; the reference itself never reads g_idx.
"""
import numpy as np


def unpack_along_k(qweight, bits):
    """(K/per, N) packed words -> (K, N) int32 codes; row k sits at bits (k % per)*bits."""
    per, mask = 32 // bits, (1 << bits) - 1
    w = np.asarray(qweight).view(np.uint32)
    out = np.empty((w.shape[0] * per, w.shape[1]), np.int32)
    for j in range(per):
        out[j::per] = (w >> np.uint32(j * bits)) & np.uint32(mask)
    return out


def unpack_along_n(qzeros, bits):
    """(G, N/per) packed words -> (G, N) int32 codes; column n at bits (n % per)*bits."""
    per, mask = 32 // bits, (1 << bits) - 1
    w = np.asarray(qzeros).view(np.uint32)
    out = np.empty((w.shape[0], w.shape[1] * per), np.int32)
    for j in range(per):
        out[:, j::per] = (w >> np.uint32(j * bits)) & np.uint32(mask)
    return out


def gptq_matmul_np(x, qweight, qzeros, scales, K, N, gs, bits, zoff=0.0, block=2048):
    """x (M, K) @ dequant(W) -> (M, N) float32, following `_gptq_matmul_np`
    (`webtorch/_core.py:4046-4072`).

    Per block of `block` output columns: unpack the codes of those columns, unpack the zero
    points, form `(scale * (q - (z + zoff)))` in float64 (exact for fp16-origin scales) and
    round it once to float32, then one float32 matmul. Groups are consecutive runs of `gs`
    rows (g = k // gs); g_idx is not consulted, as in the reference."""
    x = np.asarray(x, np.float32)
    sc = np.asarray(scales, np.float32)
    per = 32 // bits
    kp = int(np.asarray(qweight).shape[0]) * per
    grp = np.arange(kp) // gs
    out = np.empty((x.shape[0], N), np.float32)
    for c0 in range(0, N, block):
        c1 = min(N, c0 + block)
        q = unpack_along_k(np.asarray(qweight)[:, c0:c1], bits)
        # the reference unpacks every column's zero point in each block; kept for timing parity
        zb = unpack_along_n(qzeros, bits)[:, c0:c1].astype(np.float64) + float(zoff)
        w = (sc[grp, c0:c1].astype(np.float64) * (q - zb[grp])).astype(np.float32)
        out[:, c0:c1] = x @ w
    return out


def dequant_closed_form(qweight, qzeros, scales, gs, bits, zoff=0.0, g_idx=None):
    """W[k, n] = scale[g(k), n] * (q[k, n] - z[g(k), n] - zoff) as float32, g(k) = g_idx[k]
    when given (AutoGPTQ act-order), else k // gs. The product is formed in float64 and
    rounded once, which is what `_gptq_matmul_np` does for each column block."""
    q = unpack_along_k(qweight, bits)
    z = unpack_along_n(qzeros, bits).astype(np.float64) + float(zoff)
    sc = np.asarray(scales, np.float32).astype(np.float64)
    g = (np.arange(q.shape[0]) // gs) if g_idx is None else np.asarray(g_idx, np.int64)
    return (sc[g] * (q - z[g])).astype(np.float32)


def act_order_equivalent(x, qweight, g_idx, bits, gs):
    """Rewrite an act-order layer onto the plain (g = k // gs) layout: stable-sort rows by
    g_idx, permute the activation columns and repack the codes. Then the reference path
    (`gptq_matmul_np`) computes the same sum, up to float reassociation.

    Returns (x_perm, qweight_perm, perm)."""
    per = 32 // bits
    perm = np.argsort(np.asarray(g_idx), kind="stable")
    q = unpack_along_k(qweight, bits)[perm]
    K, N = q.shape
    if np.any(np.asarray(g_idx)[perm] != np.arange(K) // gs):
        raise ValueError("g_idx does not hold exactly gs rows per group")
    packed = np.zeros((K // per, N), np.uint32)
    for j in range(per):
        packed |= q[j::per].astype(np.uint32) << np.uint32(j * bits)
    return np.asarray(x)[:, perm], packed.view(np.int32), perm


def gptq_quantize(W, group_size=32, bits=4, from_out_in=False, block=2048):
    """Asymmetric min-max quantizer, following `_gptq_quantize` (`webtorch/_core.py:3782-3824`).

    W is (K, N) (or (N, K) with from_out_in). Per group of `group_size` rows and per column:
    scale = (max - min) / qmax in float32 (a zero scale becomes 1e-8), zero = clip(round(-min
    / scale)), code = clip(round(w / scale) + zero). Rounding is numpy's half-to-even in
    float32. Codes pack `per` rows per int32 along K, zeros pack along N, zero_offset is 0.
    Returns (qweight, qzeros, scales float32, K, N)."""
    W = np.asarray(W)
    K, N = (W.shape[1], W.shape[0]) if from_out_in else W.shape
    per, qmax = 32 // bits, (1 << bits) - 1
    if K % group_size or K % per or N % per:
        raise AssertionError("dims must divide group/pack size")
    G = K // group_size
    scales = np.zeros((G, N), np.float32)
    zeros = np.zeros((G, N), np.int32)
    qweight = np.zeros((K // per, N), np.uint32)
    for n0 in range(0, N, block):
        n1 = min(N, n0 + block)
        Wb = np.ascontiguousarray(W[n0:n1].T) if from_out_in else W[:, n0:n1]
        codes = np.empty((K, n1 - n0), np.int32)
        for g in range(G):
            rows = Wb[g * group_size:(g + 1) * group_size]
            lo, hi = rows.min(0), rows.max(0)
            s = (hi - lo) / qmax
            s[s == 0] = 1e-8
            z = np.clip(np.round(-lo / s), 0, qmax).astype(np.int32)
            scales[g, n0:n1] = s
            zeros[g, n0:n1] = z
            v = np.round(rows / s).astype(np.float64) + z
            codes[g * group_size:(g + 1) * group_size] = np.clip(v, 0, qmax).astype(np.int32)
        for j in range(per):
            qweight[:, n0:n1] |= codes[j::per].astype(np.uint32) << np.uint32(j * bits)
    qz = np.zeros((G, N // per), np.uint32)
    for j in range(per):
        qz |= zeros[:, j::per].astype(np.uint32) << np.uint32(j * bits)
    return qweight.view(np.int32), qz.view(np.int32), scales, K, N


def pack_autogptq(q, scale, zp, gs, bits):
    """AutoGPTQ on-disk packing (`webtorch/quantize.py:96-106`): codes along K, stored zero
    (zp - 1) & mask along N, fp16 scales, g_idx = arange // gs."""
    per, mask = 32 // bits, (1 << bits) - 1
    q = np.asarray(q, np.int64); zp = np.asarray(zp, np.int64)
    K, N = q.shape
    qweight = np.zeros((K // per, N), np.uint32)
    for j in range(per):
        qweight |= (q[j::per] & mask).astype(np.uint32) << np.uint32(j * bits)
    zs = ((zp - 1) & mask).astype(np.uint32)
    qzeros = np.zeros((zp.shape[0], N // per), np.uint32)
    for j in range(per):
        qzeros |= zs[:, j::per] << np.uint32(j * bits)
    return (qweight.view(np.int32), qzeros.view(np.int32), np.asarray(scale).astype(np.float16),
            (np.arange(K, dtype=np.int32) // gs))


def linear_forward(x, layer, zoff=1.0, g_idx=None):
    """QuantizedLinear.forward on the CPU (`webtorch/_core.py:4446-4456`) for an AutoGPTQ
    layer dict: matmul through `gptq_matmul_np`, then the float32 bias. With `g_idx` the
    act-order layer is first rewritten by `act_order_equivalent`."""
    qw, K, N = layer["qweight"], layer["K"], layer["N"]
    x = np.asarray(x, np.float32)
    if g_idx is not None:
        x, qw, _ = act_order_equivalent(x, qw, g_idx, layer["bits"], layer["gs"])
    y = gptq_matmul_np(x, qw, layer["qzeros"], layer["scales"], K, N, layer["gs"],
                       layer["bits"], zoff)
    b = layer.get("bias")
    return y if b is None else y + np.asarray(b, np.float32)
