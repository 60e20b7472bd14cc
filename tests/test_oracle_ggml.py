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
