"""Pins the Q4_K oracle (CPU) against llama.cpp's published `dequantize_row_q4_K` algorithm,
written here as scalar loops, plus special cases and the packer round trip."""
import numpy as np

from oracle import q4k
from webpytorch_amd import synth


def scalar_scale_min(s, j):
    """get_scale_min_k4 as published (llama.cpp k-quants): 6-bit pairs for j < 4, split
    nibble + 2 high bits for j >= 4."""
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)


def scalar_dequant_block(b):
    b = bytes(b)
    d = float(np.frombuffer(b[0:2], np.float16)[0])
    dmin = float(np.frombuffer(b[2:4], np.float16)[0])
    s = b[4:16]
    qs = b[16:144]
    y = np.zeros(256, np.float32)
    # 4 chunks of 64 outputs: the low nibbles of 32 code bytes, then their high nibbles
    for c in range(4):
        sc1, m1 = scalar_scale_min(s, 2 * c)
        sc2, m2 = scalar_scale_min(s, 2 * c + 1)
        d1, mm1 = np.float32(d) * np.float32(sc1), np.float32(dmin) * np.float32(m1)
        d2, mm2 = np.float32(d) * np.float32(sc2), np.float32(dmin) * np.float32(m2)
        for l in range(32):
            byte = qs[32 * c + l]
            y[64 * c + l] = np.float32(d1 * np.float32(byte & 0xF)) - mm1
            y[64 * c + 32 + l] = np.float32(d2 * np.float32(byte >> 4)) - mm2
    return y


def test_matches_scalar_published_algorithm():
    blk = synth.q4k_blocks(1, 6)
    # plus fully random bytes (any scale bits), finite fp16 fields only
    rnd = np.random.default_rng(0).integers(0, 256, (4, 144), dtype=np.uint8)
    rnd[:, 1] &= 0x3B
    rnd[:, 3] &= 0x3B
    allb = np.concatenate([blk, rnd])
    got = q4k.q4k_dequant(allb.reshape(-1), allb.shape[0] * 256).reshape(-1, 256)
    for i in range(allb.shape[0]):
        assert np.array_equal(got[i], scalar_dequant_block(allb[i])), i


def test_packer_roundtrip():
    g = np.random.default_rng(3)
    sc = g.integers(0, 64, (50, 8))
    m = g.integers(0, 64, (50, 8))
    packed = synth.pack_q4k_scales(sc, m)
    s2, m2 = q4k.scale_min_k4(packed)
    assert np.array_equal(s2, sc) and np.array_equal(m2, m)
    for i in range(5):
        for j in range(8):
            assert scalar_scale_min(bytes(packed[i]), j) == (sc[i, j], m[i, j])


def test_special_cases():
    blk = synth.q4k_blocks(2, 3)
    # d = dmin = 0 -> zeros
    z = blk.copy()
    z[:, 0:4] = 0
    assert np.all(q4k.q4k_dequant(z.reshape(-1), 3 * 256) == 0)
    # all sub-scales zero -> every value is -dmin*m[j]
    ns = blk.copy()
    sc = np.zeros((3, 8), np.int64)
    m = np.random.default_rng(1).integers(0, 64, (3, 8))
    ns[:, 4:16] = synth.pack_q4k_scales(sc, m)
    y = q4k.q4k_dequant(ns.reshape(-1), 3 * 256).reshape(3, 8, 32)
    dmin = ns[:, 2:4].copy().view(np.float16).astype(np.float32)
    assert np.array_equal(y, np.broadcast_to(-(dmin * m.astype(np.float32))[:, :, None], y.shape))
    # one nonzero code: d*sc*code - dmin*m at one spot
    one = blk[:1].copy()
    one[0, 16:] = 0
    one[0, 16 + 5] = 0x90                     # byte 5 of group 0: low 0 (sub-block 0), high 9 (sub-block 1)
    y = q4k.q4k_dequant(one.reshape(-1), 256)
    d = float(one[0, 0:2].view(np.float16)[0]); dmin = float(one[0, 2:4].view(np.float16)[0])
    sc, m = q4k.scale_min_k4(one[:, 4:16])
    assert y[32 + 5] == np.float32(np.float32(d) * sc[0, 1] * 9) - np.float32(np.float32(dmin) * m[0, 1])
    assert y[5] == -np.float32(np.float32(dmin) * m[0, 0])


def test_matmul_brute_force():
    K, N, M = 512, 6, 2
    W = synth.q4k_layer(4, K, N)
    x = synth.activations(4, M, K, np.float32)
    rows = np.stack([np.concatenate([scalar_dequant_block(W[n, 144 * b:144 * (b + 1)]) for b in range(K // 256)])
                     for n in range(N)])
    ref = x.astype(np.float64) @ rows.T.astype(np.float64)
    got = q4k.q4k_matmul(x, W, K, N)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
