"""The Q8_0 / Q6_K oracle against a scalar, per-element restatement of llama.cpp's published
dequantization loops, special cases, and a float64 brute-force matmul."""
import struct

import numpy as np
import pytest

from oracle import ggml
from webpytorch_amd import synth


def _half(b, o):
    return float(np.frombuffer(bytes(b[o:o + 2]), np.float16)[0])


def scalar_q8_0(raw, n):
    """dequantize_row_q8_0: y[i*32 + j] = d * qs[j]."""
    out = []
    for i in range(n // 32):
        blk = raw[34 * i:34 * (i + 1)]
        d = _half(blk, 0)
        for j in range(32):
            out.append(np.float32(d) * np.float32(struct.unpack("b", bytes([blk[2 + j]]))[0]))
    return np.array(out, np.float32)


def scalar_q6k(raw, n):
    """dequantize_row_q6_K: per 128-weight half, pointers ql += 64, qh += 32, sc += 8; for l <
    32 with is = l / 16 the four weights y[l + 32 k] use ql[l] / ql[l + 32] nibbles and qh[l]
    bit pairs, scales sc[is + 2 k]."""
    out = np.zeros(n, np.float32)
    for i in range(n // 256):
        blk = raw[210 * i:210 * (i + 1)]
        d = np.float32(_half(blk, 208))
        ql, qh, sc = 0, 128, 192
        y = 256 * i
        for _ in range(2):
            for l in range(32):
                is_ = l // 16
                q1 = ((blk[ql + l] & 0xF) | (((blk[qh + l] >> 0) & 3) << 4)) - 32
                q2 = ((blk[ql + l + 32] & 0xF) | (((blk[qh + l] >> 2) & 3) << 4)) - 32
                q3 = ((blk[ql + l] >> 4) | (((blk[qh + l] >> 4) & 3) << 4)) - 32
                q4 = ((blk[ql + l + 32] >> 4) | (((blk[qh + l] >> 6) & 3) << 4)) - 32
                s = [np.float32(struct.unpack("b", bytes([blk[sc + is_ + 2 * k]]))[0]) for k in range(4)]
                out[y + l] = d * s[0] * np.float32(q1)
                out[y + l + 32] = d * s[1] * np.float32(q2)
                out[y + l + 64] = d * s[2] * np.float32(q3)
                out[y + l + 96] = d * s[3] * np.float32(q4)
            ql += 64
            qh += 32
            sc += 8
            y += 128
    return out


@pytest.mark.parametrize("seed", [0, 1])
def test_q8_0_matches_published_loop(seed):
    W = synth.q8_0_layer(seed, 128, 3)
    raw = W.tobytes()
    assert np.array_equal(ggml.q8_0_dequant(raw, 384), scalar_q8_0(raw, 384))


@pytest.mark.parametrize("seed", [0, 1])
def test_q6k_matches_published_loop(seed):
    W = synth.q6k_layer(seed, 512, 2)
    raw = W.tobytes()
    assert np.array_equal(ggml.q6k_dequant(raw, 1024), scalar_q6k(raw, 1024))


def test_special_cases():
    one = np.array([1.0], np.float16).view(np.uint8)
    # Q8_0: d = 0 -> zeros; d = 1 -> the signed bytes themselves
    b = np.zeros(34, np.uint8)
    b[2:] = np.arange(-16, 16).astype(np.int8).view(np.uint8)
    assert not ggml.q8_0_dequant(b.tobytes(), 32).any()
    b[0:2] = one
    assert np.array_equal(ggml.q8_0_dequant(b.tobytes(), 32), np.arange(-16, 16, dtype=np.float32))
    # Q6_K: d = 1, unit scales, zero codes -> -32 everywhere
    q = np.zeros(210, np.uint8)
    q[192:208] = 1
    q[208:210] = one
    assert np.array_equal(ggml.q6k_dequant(q.tobytes(), 256), np.full(256, -32, np.float32))
    # one ql byte (index 5 of half 0) = 0xA3: weight 5 (low nibble 3) and weight 69 (high nibble 10)
    q2 = q.copy()
    q2[5] = 0xA3
    v = ggml.q6k_dequant(q2.tobytes(), 256)
    want = np.full(256, -32, np.float32)
    want[5], want[69] = 3 - 32, 10 - 32
    assert np.array_equal(v, want)
    # one qh byte (index 40 = half 1, l = 8) = 0b11_10_01_00: bits feed weights 136, 168, 200, 232
    q3 = q.copy()
    q3[128 + 40] = 0b11100100
    v = ggml.q6k_dequant(q3.tobytes(), 256)
    want = np.full(256, -32, np.float32)
    want[[136, 168, 200, 232]] = np.array([0, 16, 32, 48], np.float32) - 32
    assert np.array_equal(v, want)
    # scale byte 8 + 1 + 2 * 3 = 15 (half 1, l in 16..31, k = 3) = -2: weights 128 + 96 + 16..31
    q4 = q.copy()
    q4[192 + 15] = np.int8(-2).view(np.uint8)
    v = ggml.q6k_dequant(q4.tobytes(), 256)
    want = np.full(256, -32, np.float32)
    want[128 + 96 + 16:128 + 96 + 32] = 64
    assert np.array_equal(v, want)


@pytest.mark.parametrize("type_name,K,N", [("Q8_0", 96, 5), ("Q6_K", 512, 3)])
def test_matmul_brute_force(type_name, K, N):
    W = (synth.q8_0_layer if type_name == "Q8_0" else synth.q6k_layer)(7, K, N)
    x = synth.activations(7, 2, K, np.float32)
    got = ggml.ggml_matmul(x, W, type_name, K, N)
    Wd = (scalar_q8_0 if type_name == "Q8_0" else scalar_q6k)(W.tobytes(), N * K).reshape(N, K)
    ref = x.astype(np.float64) @ Wd.astype(np.float64).T
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


# ---- the other block types: scalar restatements of llama.cpp's dequantize_row_* loops --------

KV = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]  # kvalues_iq4nl
F = np.float32


def _u16(b, o):
    return int(b[o]) | (int(b[o + 1]) << 8)


def _u32(b, o):
    return _u16(b, o) | (_u16(b, o + 2) << 16)


def scalar_q4_0(raw, n):
    """y[j] = (qs[j] & 0xF) - 8, y[j + 16] = (qs[j] >> 4) - 8, each times d."""
    out = np.zeros(n, F)
    for i in range(n // 32):
        b = raw[18 * i:18 * i + 18]
        d = F(_half(b, 0))
        for j in range(16):
            out[32 * i + j] = F((b[2 + j] & 0xF) - 8) * d
            out[32 * i + j + 16] = F((b[2 + j] >> 4) - 8) * d
    return out


def scalar_q4_1(raw, n):
    out = np.zeros(n, F)
    for i in range(n // 32):
        b = raw[20 * i:20 * i + 20]
        d, m = F(_half(b, 0)), F(_half(b, 2))
        for j in range(16):
            out[32 * i + j] = F(b[4 + j] & 0xF) * d + m
            out[32 * i + j + 16] = F(b[4 + j] >> 4) * d + m
    return out


def scalar_q5(raw, n, with_min):
    """q5_0 / q5_1: xh_0 = ((qh >> j) << 4) & 0x10, xh_1 = (qh >> (j + 12)) & 0x10."""
    sz = 24 if with_min else 22
    out = np.zeros(n, F)
    for i in range(n // 32):
        b = raw[sz * i:sz * i + sz]
        d = F(_half(b, 0))
        m = F(_half(b, 2)) if with_min else None
        o = 4 if with_min else 2
        qh = _u32(b, o)
        for j in range(16):
            xh0 = ((qh >> j) << 4) & 0x10
            xh1 = (qh >> (j + 12)) & 0x10
            x0 = (b[o + 4 + j] & 0x0F) | xh0
            x1 = (b[o + 4 + j] >> 4) | xh1
            if with_min:
                out[32 * i + j] = F(x0) * d + m
                out[32 * i + j + 16] = F(x1) * d + m
            else:
                out[32 * i + j] = F(x0 - 16) * d
                out[32 * i + j + 16] = F(x1 - 16) * d
    return out


def scalar_iq4_nl(raw, n):
    out = np.zeros(n, F)
    for i in range(n // 32):
        b = raw[18 * i:18 * i + 18]
        d = F(_half(b, 0))
        for j in range(16):
            out[32 * i + j] = d * F(KV[b[2 + j] & 0xF])
            out[32 * i + j + 16] = d * F(KV[b[2 + j] >> 4])
    return out


def scalar_iq4_xs(raw, n):
    out = np.zeros(n, F)
    for i in range(n // 256):
        b = raw[136 * i:136 * i + 136]
        d = F(_half(b, 0))
        sh = _u16(b, 2)
        y = 256 * i
        for ib in range(8):
            ls = ((b[4 + ib // 2] >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4)
            dl = d * F(ls - 32)
            q = 8 + 16 * ib
            for j in range(16):
                out[y + j] = dl * F(KV[b[q + j] & 0xF])
                out[y + j + 16] = dl * F(KV[b[q + j] >> 4])
            y += 32
    return out


def get_scale_min_k4(j, q):
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def scalar_q5k(raw, n):
    out = np.zeros(n, F)
    for i in range(n // 256):
        b = raw[176 * i:176 * i + 176]
        d, mn = F(_half(b, 0)), F(_half(b, 2))
        sc = b[4:16]
        y, ql, is_, u1, u2 = 256 * i, 48, 0, 1, 2
        for _ in range(4):
            s1, m1 = get_scale_min_k4(is_, sc)
            s2, m2 = get_scale_min_k4(is_ + 1, sc)
            d1, mm1, d2, mm2 = d * F(s1), mn * F(m1), d * F(s2), mn * F(m2)
            for l in range(32):
                out[y + l] = d1 * F((b[ql + l] & 0xF) + (16 if b[16 + l] & u1 else 0)) - mm1
            for l in range(32):
                out[y + 32 + l] = d2 * F((b[ql + l] >> 4) + (16 if b[16 + l] & u2 else 0)) - mm2
            y += 64
            ql += 32
            is_ += 2
            u1 <<= 2
            u2 <<= 2
    return out


def scalar_q2k(raw, n):
    out = np.zeros(n, F)
    for i in range(n // 256):
        b = raw[84 * i:84 * i + 84]
        d, mn = F(_half(b, 80)), F(_half(b, 82))
        y, q, is_ = 256 * i, 16, 0
        for _ in range(2):
            shift = 0
            for _ in range(4):
                for half in range(2):
                    sc = b[is_]
                    is_ += 1
                    dl, ml = d * F(sc & 0xF), mn * F(sc >> 4)
                    for l in range(16):
                        out[y] = dl * F((b[q + 16 * half + l] >> shift) & 3) - ml
                        y += 1
                shift += 2
            q += 32
    return out


def scalar_q3k(raw, n):
    """With the scales unpacked the way llama.cpp does it: the 12 bytes as three 32-bit words,
    rebuilt into four words of 6-bit values by the kmask1 / kmask2 shifts."""
    k1, k2 = 0x03030303, 0x0F0F0F0F
    out = np.zeros(n, F)
    for i in range(n // 256):
        b = raw[110 * i:110 * i + 110]
        d = F(_half(b, 108))
        a = [_u32(b, 96), _u32(b, 100), _u32(b, 104)]
        tmp = a[2]
        aux = [(a[0] & k2) | (((tmp >> 0) & k1) << 4), (a[1] & k2) | (((tmp >> 2) & k1) << 4),
               ((a[0] >> 4) & k2) | (((tmp >> 4) & k1) << 4), ((a[1] >> 4) & k2) | (((tmp >> 6) & k1) << 4)]
        scales = [((aux[k // 4] >> (8 * (k % 4))) & 0xFF) for k in range(16)]
        scales = [s - 256 if s >= 128 else s for s in scales]
        y, q, m, is_ = 256 * i, 32, 1, 0
        for _ in range(2):
            shift = 0
            for _ in range(4):
                for half in range(2):
                    dl = d * F(scales[is_] - 32)
                    is_ += 1
                    for l in range(16):
                        v = ((b[q + 16 * half + l] >> shift) & 3) - (0 if b[16 * half + l] & m else 4)
                        out[y] = dl * F(v)
                        y += 1
                shift += 2
                m <<= 1
            q += 32
    return out


SCALAR = {"Q4_0": scalar_q4_0, "Q4_1": scalar_q4_1, "Q5_0": lambda r, n: scalar_q5(r, n, False),
          "Q5_1": lambda r, n: scalar_q5(r, n, True), "IQ4_NL": scalar_iq4_nl, "IQ4_XS": scalar_iq4_xs,
          "Q5_K": scalar_q5k, "Q2_K": scalar_q2k, "Q3_K": scalar_q3k}


def _random_blocks(type_name, nblocks, seed):
    """Random bytes with finite fp16 fields (exponent kept below Inf/NaN)."""
    vals, nbytes = ggml.DEQUANT[type_name][1:]
    b = np.random.default_rng(seed).integers(0, 256, (nblocks, nbytes), dtype=np.uint8)
    for off in ggml.F16_FIELDS[type_name]:
        b[:, off + 1] &= 0x3B
    return b


@pytest.mark.parametrize("type_name", sorted(SCALAR))
@pytest.mark.parametrize("seed", [0, 1])
def test_block_types_match_published_loops(type_name, seed):
    vals = ggml.DEQUANT[type_name][1]
    raw = _random_blocks(type_name, 3, seed).reshape(-1)
    got = ggml.DEQUANT[type_name][0](raw.tobytes(), 3 * vals)
    want = SCALAR[type_name](raw.tobytes(), 3 * vals)  # bytes index to Python ints (no uint8 wrap)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("type_name", sorted(SCALAR))
def test_block_types_special_cases(type_name):
    """Zero fp16 fields give zeros; one changed code byte moves only the weights it feeds."""
    vals, nbytes = ggml.DEQUANT[type_name][1:]
    f = ggml.DEQUANT[type_name][0]
    b = _random_blocks(type_name, 2, 7)
    z = b.copy()
    for off in ggml.F16_FIELDS[type_name]:
        z[:, off:off + 2] = 0
    assert not np.any(f(z.reshape(-1).tobytes(), 2 * vals))
    base = f(b.reshape(-1).tobytes(), 2 * vals)
    c = b.copy()
    qoff = ggml.CODE_BYTES[type_name]
    c[1, qoff] ^= 0xFF
    moved = np.nonzero(f(c.reshape(-1).tobytes(), 2 * vals) != base)[0]
    assert moved.size and moved.min() >= vals and moved.size <= 8  # only block 1, one byte's weights


def test_q4_1_and_iq4_unit_scale_values():
    """d = 1 and m = 0 give the raw codes (Q4_1) or the codebook (IQ4_NL)."""
    one = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    b = np.zeros(20, np.uint8)
    b[0:2] = one
    b[4:20] = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
    got = ggml.q4_1_dequant(b.tobytes(), 32)
    assert np.array_equal(got, np.concatenate([np.arange(16), np.arange(16)[::-1]]).astype(F))
    b = np.zeros(18, np.uint8)
    b[0:2] = one
    b[2:18] = np.arange(16, dtype=np.uint8)
    assert np.array_equal(ggml.iq4_nl_dequant(b.tobytes(), 32)[:16], np.array(KV, F))
