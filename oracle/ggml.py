"""GGUF block-type oracle beside Q4_K (test infrastructure only; see `oracle/__init__.py`).

Follows `ggufload.dequant` (`webtorch/ggufload.py:133-300`) for Q8_0, Q4_0, Q4_1, Q5_0, Q5_1,
IQ4_NL, IQ4_XS, Q2_K, Q3_K, Q5_K and Q6_K, and the `UnquantizedLinear` float32 matmul
(`webtorch/_core.py:4462-4481`) that the reference uses for a dequantized GGUF weight on the CPU.
Every value is one float32 rounding of an exact product (fp16 scale, small integer sub-scale
and code: at most 24 significant bits), or of such a product minus/plus another exact one
(the Q4_1 / Q5_1 min, the K-quant mins), so any evaluation order with products first gives the
same bits.

Pins (tests/test_oracle_ggml.py): a scalar, per-element restatement of llama.cpp's published
`dequantize_row_*` loop of each type (index arithmetic written independently of the vectorized
forms below); special cases (d = 0 gives zeros; unit scales give the raw codes or codebook
values; one nonzero byte moves exactly the weights that byte feeds); the matmul against a
float64 brute force.
"""
import numpy as np

Q8_0_VALS, Q8_0_BYTES = 32, 34
Q6K_VALS, Q6K_BYTES = 256, 210


def _u8(raw):
    return np.frombuffer(raw if isinstance(raw, (bytes, bytearray)) else np.ascontiguousarray(raw).tobytes(),
                         np.uint8)


def _f16(b):
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32)


def q8_0_dequant(raw, n):
    """First n values of a Q8_0 byte stream: d * q, d the block's leading fp16."""
    nb = n // Q8_0_VALS
    b = _u8(raw)[:nb * Q8_0_BYTES].reshape(nb, Q8_0_BYTES)
    d = _f16(b[:, 0:2])                                   # (nb, 1)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d * q).reshape(-1)[:n]


def q6k_dequant(raw, n):
    """First n values of a Q6_K byte stream. Half h of a super-block takes ql[64h:64h+64],
    qh[32h:32h+32] and scales[8h:8h+8]; weight 128h + 32j + l has the 6-bit code made of the
    low (j < 2) or high (j >= 2) nibble of ql[64h + l + 32 (j % 2)] and bits 2j, 2j+1 of
    qh[32h + l], scale scales[8h + l // 16 + 2j], value d * scale * (code - 32)."""
    nb = n // Q6K_VALS
    b = _u8(raw)[:nb * Q6K_BYTES].reshape(nb, Q6K_BYTES)
    ql, qh = b[:, 0:128].astype(np.int32), b[:, 128:192].astype(np.int32)
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    d = _f16(b[:, 208:210])                               # (nb, 1)
    out = np.empty((nb, 2, 4, 32), np.float32)
    l = np.arange(32)
    for h in range(2):
        for j in range(4):
            lo = ql[:, 64 * h + 32 * (j % 2) + l]
            nib = (lo & 15) if j < 2 else (lo >> 4)
            code = nib | (((qh[:, 32 * h + l] >> (2 * j)) & 3) << 4)
            scale = sc[:, 8 * h + l // 16 + 2 * j]
            out[:, h, j, :] = (d * scale) * (code - 32).astype(np.float32)
    return out.reshape(-1)[:n]


# the IQ4_NL / IQ4_XS codebook (`webtorch/ggufload.py:32-33`, llama.cpp's kvalues_iq4nl)
IQ4NL_VALUES = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)


def _blocks(raw, n, vals, nbytes):
    nb = n // vals
    return _u8(raw)[:nb * nbytes].reshape(nb, nbytes)


def _nibbles32(qs):
    """(nb, 16) bytes -> (nb, 32) codes: the low nibbles are values 0-15, the high 16-31."""
    qs = qs.astype(np.int32)
    return np.concatenate([qs & 15, qs >> 4], axis=1)


def q4_0_dequant(raw, n):
    """32 values / 18 bytes: fp16 d, 16 nibble pairs; d * (q - 8)."""
    b = _blocks(raw, n, 32, 18)
    return (_f16(b[:, 0:2]) * (_nibbles32(b[:, 2:18]) - 8).astype(np.float32)).reshape(-1)[:n]


def q4_1_dequant(raw, n):
    """32 values / 20 bytes: fp16 d, fp16 m, 16 nibble pairs; d * q + m."""
    b = _blocks(raw, n, 32, 20)
    return (_f16(b[:, 0:2]) * _nibbles32(b[:, 4:20]).astype(np.float32) + _f16(b[:, 2:4])).reshape(-1)[:n]


def _fifth_bits(qh):
    """(nb, 4) bytes of the 32-bit fifth-bit word -> (nb, 32) values 0 or 16: value j < 16 takes
    bit j, value 16 + j bit j + 16."""
    w = np.ascontiguousarray(qh).view(np.uint32).reshape(-1, 1).astype(np.int64)
    return (((w >> np.arange(32)) & 1) << 4).astype(np.int32)


def q5_0_dequant(raw, n):
    """32 values / 22 bytes: fp16 d, u32 fifth bits, 16 nibble pairs; d * (q - 16)."""
    b = _blocks(raw, n, 32, 22)
    q = _nibbles32(b[:, 6:22]) | _fifth_bits(b[:, 2:6])
    return (_f16(b[:, 0:2]) * (q - 16).astype(np.float32)).reshape(-1)[:n]


def q5_1_dequant(raw, n):
    """32 values / 24 bytes: fp16 d, fp16 m, u32 fifth bits, 16 nibble pairs; d * q + m."""
    b = _blocks(raw, n, 32, 24)
    q = _nibbles32(b[:, 8:24]) | _fifth_bits(b[:, 4:8])
    return (_f16(b[:, 0:2]) * q.astype(np.float32) + _f16(b[:, 2:4])).reshape(-1)[:n]


def iq4_nl_dequant(raw, n):
    """32 values / 18 bytes: fp16 d, 16 nibble pairs indexing the codebook; d * kv[q]."""
    b = _blocks(raw, n, 32, 18)
    return (_f16(b[:, 0:2]) * IQ4NL_VALUES[_nibbles32(b[:, 2:18])]).reshape(-1)[:n]


def iq4_xs_dequant(raw, n):
    """256 values / 136 bytes: fp16 d, u16 high scale bits, 4 bytes of low scale nibbles,
    128 bytes of codebook nibbles. Sub-block ib (32 values): ls = low nibble ib of the scales_l
    bytes | two bits 2 ib of scales_h << 4; (d * (ls - 32)) * kv[q], codes as IQ4_NL."""
    b = _blocks(raw, n, 256, 136)
    nb = b.shape[0]
    d = _f16(b[:, 0:2])
    sh = b[:, 2].astype(np.int32) | (b[:, 3].astype(np.int32) << 8)
    ib = np.arange(8)
    low = (b[:, 4 + ib // 2].astype(np.int32) >> (4 * (ib % 2))) & 15
    ls = low | (((sh[:, None] >> (2 * ib)) & 3) << 4)
    dl = d * (ls - 32).astype(np.float32)                                     # (nb, 8)
    codes = _nibbles32(b[:, 8:136].reshape(nb * 8, 16)).reshape(nb, 8, 32)
    return (dl[:, :, None] * IQ4NL_VALUES[codes]).reshape(-1)[:n]


def _k4_scales(s):
    """The 12-byte 6-bit scale/min packing of Q4_K / Q5_K (`get_scale_min_k4`)."""
    s = np.asarray(s, np.int32)
    sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)], axis=1)
    mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
    return sc.astype(np.float32), mn.astype(np.float32)


def q5k_dequant(raw, n):
    """256 values / 176 bytes: fp16 d, fp16 dmin, 12 bytes of scales/mins, qh[32], qs[128].
    Group g (64 values): sub-block 2g = low nibbles of qs[32g:32g+32] + 16 * bit 2g of qh[l],
    sub-block 2g+1 = high nibbles + 16 * bit 2g+1; (d * sc) * q - dmin * m."""
    b = _blocks(raw, n, 256, 176)
    nb = b.shape[0]
    d, dmin = _f16(b[:, 0:2]), _f16(b[:, 2:4])
    sc, mn = _k4_scales(b[:, 4:16])
    qh = b[:, 16:48].astype(np.int32)
    qs = b[:, 48:176].astype(np.int32).reshape(nb, 4, 32)
    out = np.empty((nb, 8, 32), np.float32)
    for j in range(8):
        g, hi = j // 2, j % 2
        q = ((qs[:, g] >> (4 * hi)) & 15) + 16 * ((qh >> j) & 1)
        out[:, j] = (d * sc[:, j:j + 1]) * q.astype(np.float32) - dmin * mn[:, j:j + 1]
    return out.reshape(-1)[:n]


def q2k_dequant(raw, n):
    """256 values / 84 bytes: scales[16] (low nibble scale, high nibble min), qs[64], fp16 d,
    fp16 dmin. Value 128 h + 32 j + 16 u + l (h < 2, j < 4, u < 2, l < 16) is bits 2j of
    qs[32 h + 16 u + l] with scale byte 8 h + 2 j + u: (d * sc) * q - dmin * m."""
    b = _blocks(raw, n, 256, 84)
    nb = b.shape[0]
    d, dmin = _f16(b[:, 80:82]), _f16(b[:, 82:84])
    out = np.empty((nb, 2, 4, 2, 16), np.float32)
    for h in range(2):
        for j in range(4):
            for u in range(2):
                s = b[:, 8 * h + 2 * j + u].astype(np.int32)
                q = (b[:, 16 + 32 * h + 16 * u:16 + 32 * h + 16 * u + 16].astype(np.int32) >> (2 * j)) & 3
                out[:, h, j, u] = (d * (s & 15)[:, None].astype(np.float32)) * q.astype(np.float32) - \
                    dmin * (s >> 4)[:, None].astype(np.float32)
    return out.reshape(-1)[:n]


def q3k_scales(s):
    """The 12 bytes of Q3_K scales -> (nb, 16) signed scales (6 bits, minus 32): scale i has low
    nibble from byte i mod 8 (its low nibble for i < 8, high for i >= 8) and two high bits from
    byte 8 + i mod 4 at bit pair i // 4."""
    s = np.asarray(s, np.int32)
    i = np.arange(16)
    low = (s[:, i % 8] >> (4 * (i // 8))) & 15
    high = (s[:, 8 + i % 4] >> (2 * (i // 4))) & 3
    return ((low | (high << 4)) - 32).astype(np.float32)


def q3k_dequant(raw, n):
    """256 values / 110 bytes: hmask[32], qs[64], 12 bytes of scales, fp16 d. Value
    128 h + 32 j + 16 u + l: bits 2j of qs[32 h + 16 u + l] minus 4 unless bit 4 h + j of
    hmask[16 u + l] is set, times d * scale[8 h + 2 j + u]."""
    b = _blocks(raw, n, 256, 110)
    nb = b.shape[0]
    d = _f16(b[:, 108:110])
    sc = q3k_scales(b[:, 96:108])
    out = np.empty((nb, 2, 4, 2, 16), np.float32)
    for h in range(2):
        for j in range(4):
            for u in range(2):
                q = (b[:, 32 + 32 * h + 16 * u:32 + 32 * h + 16 * u + 16].astype(np.int32) >> (2 * j)) & 3
                hm = (b[:, 16 * u:16 * u + 16].astype(np.int32) >> (4 * h + j)) & 1
                out[:, h, j, u] = (d * sc[:, 8 * h + 2 * j + u:8 * h + 2 * j + u + 1]) * (q - 4 * (1 - hm)).astype(np.float32)
    return out.reshape(-1)[:n]


DEQUANT = {"Q8_0": (q8_0_dequant, Q8_0_VALS, Q8_0_BYTES), "Q6_K": (q6k_dequant, Q6K_VALS, Q6K_BYTES),
           "Q4_0": (q4_0_dequant, 32, 18), "Q4_1": (q4_1_dequant, 32, 20), "Q5_0": (q5_0_dequant, 32, 22),
           "Q5_1": (q5_1_dequant, 32, 24), "IQ4_NL": (iq4_nl_dequant, 32, 18),
           "IQ4_XS": (iq4_xs_dequant, 256, 136), "Q5_K": (q5k_dequant, 256, 176), "Q2_K": (q2k_dequant, 256, 84),
           "Q3_K": (q3k_dequant, 256, 110)}


def ggml_matmul(x, rows_bytes, type_name, K, N):
    """x (M, K) @ dequant(W).T -> (M, N) float32, W being N rows of K / block-values blocks."""
    f, vals, nbytes = DEQUANT[type_name]
    W = f(np.asarray(rows_bytes, np.uint8).reshape(-1), N * K).reshape(N, K)
    return np.asarray(x, np.float32) @ W.T


# byte offsets of each type's fp16 fields, and of one code byte (tests use them to build blocks)
F16_FIELDS = {"Q8_0": (0,), "Q6_K": (208,), "Q4_0": (0,), "Q4_1": (0, 2), "Q5_0": (0,), "Q5_1": (0, 2),
              "IQ4_NL": (0,), "IQ4_XS": (0,), "Q5_K": (0, 2), "Q2_K": (80, 82), "Q3_K": (108,)}
CODE_BYTES = {"Q8_0": 2, "Q6_K": 0, "Q4_0": 2, "Q4_1": 4, "Q5_0": 6, "Q5_1": 8, "IQ4_NL": 2, "IQ4_XS": 8,
              "Q5_K": 48, "Q2_K": 16, "Q3_K": 32}


# the types beyond the K-quants (i-quant grids, ternary, fp4, 1/2-bit, unquantized matrices)
from . import ggml_ext as _ext  # noqa: E402

for _name, _f in _ext.DEQUANT.items():
    DEQUANT[_name] = (_f,) + _ext.BLOCKS[_name]
F16_FIELDS.update(_ext.F16_FIELDS)
