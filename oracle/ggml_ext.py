"""GGUF block types beyond the K-quants (test infrastructure only; see `oracle/__init__.py`):
the codebook-grid i-quants IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M, the ternary
TQ1_0 / TQ2_0, the fp4 MXFP4 / NVFP4, the 1- and 2-bit Q1_0 / Q2_0, and the unquantized F32 /
F16 / BF16 matrices.

Follows `ggufload.dequant` / `_dequant_iq` (`webtorch/ggufload.py:302-384, 387-505`), which
transcribe llama.cpp's `dequantize_row_iq2_xxs` .. `dequantize_row_iq1_m`,
`dequantize_row_tq1_0` / `tq2_0`, `dequantize_row_mxfp4` / `nvfp4`; the loops here are written
from those published routines block field by block field (sub-block ib, group l, value j),
vectorized over blocks only. Every value is one float32 rounding of an exact product (fp16
scale times a small odd integer or a power of two, codebook entries of at most 6 bits, +-1/8
offsets), so any evaluation order gives the same bits.

The codebooks are the format's tables, read from the header the kernels compile
(`webpytorch_amd/csrc/iq_grids.h`, written by `gen_iq_grids.py` from the reference's
`webtorch/iqtables.py`); its SHA-256 digests of the values are checked against the ones taken
from the reference's tables (tests/test_oracle_ggml_ext.py).

Pins: reference-written dequant vectors of random blocks for every type
(tests/golden/ggml_ext.npz, `ggufload.dequant` run in the build container), special cases
(d = 0 gives zeros; a unit scale gives the raw grid values; one index / sign / scale byte moves
exactly the values it feeds) and the table digests.
"""
import os
import re

import numpy as np

HEADER = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "webpytorch_amd", "csrc", "iq_grids.h")

# (values per block, bytes per block) -- the ggml block sizes
BLOCKS = {"IQ2_XXS": (256, 66), "IQ2_XS": (256, 74), "IQ2_S": (256, 82), "IQ3_XXS": (256, 98),
          "IQ3_S": (256, 110), "IQ1_S": (256, 50), "IQ1_M": (256, 56), "TQ1_0": (256, 54), "TQ2_0": (256, 66),
          "MXFP4": (32, 17), "NVFP4": (64, 36), "Q1_0": (128, 18), "Q2_0": (64, 18),
          "F32": (1, 4), "F16": (1, 2), "BF16": (1, 2)}
# byte offsets of the fp16 fields (tests and the synthetic writer keep them finite)
F16_FIELDS = {"IQ2_XXS": (0,), "IQ2_XS": (0,), "IQ2_S": (0,), "IQ3_XXS": (0,), "IQ3_S": (0,), "IQ1_S": (0,),
              "IQ1_M": (), "TQ1_0": (52,), "TQ2_0": (64,), "MXFP4": (), "NVFP4": (), "Q1_0": (0,), "Q2_0": (0,)}

_GRIDS = None


def grids():
    """{name: int array (entries, values)} of the codebooks in the kernels' header."""
    global _GRIDS
    if _GRIDS is None:
        text = open(HEADER).read()
        g = {}
        for name, per in (("kIQ2XXS", 8), ("kIQ2XS", 8), ("kIQ2S", 8), ("kIQ3XXS", 4), ("kIQ3S", 4), ("kIQ1S", 8)):
            body = re.search(r"\b%s\[(\d+)\] = \{(.*?)\};" % name, text, re.S)
            vals = [int(v, 16) for v in re.findall(r"0x([0-9a-fA-F]+)", body.group(2))]
            assert len(vals) == int(body.group(1))
            if name == "kIQ1S":  # 2 bits per value, stored as value + 1
                e = np.array(vals, np.int64)[:, None]
                g[name] = (((e >> (2 * np.arange(8))) & 3) - 1).astype(np.int8)
            else:
                dt = np.uint64 if per == 8 else np.uint32
                g[name] = np.array(vals, dt).view(np.uint8).reshape(-1, per).astype(np.int32)
        _GRIDS = g
    return _GRIDS


def _u8(raw):
    return np.frombuffer(raw if isinstance(raw, (bytes, bytearray)) else np.ascontiguousarray(raw).tobytes(),
                         np.uint8)


def _blocks(raw, n, name):
    vals, nbytes = BLOCKS[name]
    nb = n // vals
    return _u8(raw)[:nb * nbytes].reshape(nb, nbytes).astype(np.int64)


def _f16(b, o):
    """(nb,) float32 of the fp16 at byte o of each block row b (int64 bytes)."""
    u = (b[:, o] | (b[:, o + 1] << 8)).astype(np.uint16)
    return u.view(np.float16).astype(np.float32)


def _u16(b, o):
    return b[:, o] | (b[:, o + 1] << 8)


def _u32(b, o):
    return b[:, o] | (b[:, o + 1] << 8) | (b[:, o + 2] << 16) | (b[:, o + 3] << 24)


def ksigns(s):
    """The sign byte a 7-bit index stands for: s with its parity as bit 7 (ggml's ksigns_iq2xs)."""
    s = np.asarray(s, np.int64)
    par = np.zeros_like(s)
    for k in range(7):
        par ^= (s >> k) & 1
    return s | (par << 7)


def _signs(mask):
    """(..., ) sign bytes -> (..., 8) float32 factors: bit j set negates value j."""
    m = np.asarray(mask, np.int64)[..., None]
    return np.where((m >> np.arange(8)) & 1, np.float32(-1.0), np.float32(1.0)).astype(np.float32)


def iq2_xxs_dequant(raw, n):
    """dequantize_row_iq2_xxs: per sub-block ib, aux32[0] = qs[4 ib] (four grid indices as
    bytes), aux32[1] = four 7-bit sign indices and a 4-bit scale; db = d (0.5 + scale) / 4;
    y[32 ib + 8 l + j] = db * grid[aux8[l]][j] * sign(ksigns[(aux32[1] >> 7 l) & 127], j)."""
    b = _blocks(raw, n, "IQ2_XXS")
    d, G = _f16(b, 0), grids()["kIQ2XXS"]
    out = np.empty((b.shape[0], 8, 4, 8), np.float32)
    for ib in range(8):
        a0, a1 = _u32(b, 2 + 8 * ib), _u32(b, 6 + 8 * ib)
        db = d * (np.float32(0.5) + (a1 >> 28).astype(np.float32)) * np.float32(0.25)
        for l in range(4):
            v = G[(a0 >> (8 * l)) & 255].astype(np.float32) * _signs(ksigns((a1 >> (7 * l)) & 127))
            out[:, ib, l] = db[:, None] * v
    return out.reshape(-1)[:n]


def iq2_xs_dequant(raw, n):
    """dequantize_row_iq2_xs: 32 u16 codes (grid index q & 511, sign index q >> 9) and 8 scale
    bytes; groups 0-1 of sub-block ib take the low nibble, 2-3 the high one."""
    b = _blocks(raw, n, "IQ2_XS")
    d, G = _f16(b, 0), grids()["kIQ2XS"]
    out = np.empty((b.shape[0], 8, 4, 8), np.float32)
    for ib in range(8):
        sc = b[:, 66 + ib]
        for l in range(4):
            q = _u16(b, 2 + 2 * (4 * ib + l))
            db = d * (np.float32(0.5) + ((sc >> (4 * (l // 2))) & 15).astype(np.float32)) * np.float32(0.25)
            out[:, ib, l] = db[:, None] * (G[q & 511].astype(np.float32) * _signs(ksigns(q >> 9)))
    return out.reshape(-1)[:n]


def iq2_s_dequant(raw, n):
    """dequantize_row_iq2_s: index qs[4 ib + l] | ((qh[ib] << (8 - 2 l)) & 0x300); the sign byte
    is qs[32 + 4 ib + l] itself; scales as IQ2_XS."""
    b = _blocks(raw, n, "IQ2_S")
    d, G = _f16(b, 0), grids()["kIQ2S"]
    out = np.empty((b.shape[0], 8, 4, 8), np.float32)
    for ib in range(8):
        qh, sc = b[:, 66 + ib], b[:, 74 + ib]
        for l in range(4):
            idx = b[:, 2 + 4 * ib + l] | ((qh << (8 - 2 * l)) & 0x300)
            db = d * (np.float32(0.5) + ((sc >> (4 * (l // 2))) & 15).astype(np.float32)) * np.float32(0.25)
            out[:, ib, l] = db[:, None] * (G[idx].astype(np.float32) * _signs(b[:, 34 + 4 * ib + l]))
    return out.reshape(-1)[:n]


def iq3_xxs_dequant(raw, n):
    """dequantize_row_iq3_xxs: 64 grid index bytes (entries of 4 values, two per group), then one
    u32 per sub-block with four 7-bit sign indices and a 4-bit scale; db = d (0.5 + scale) / 2."""
    b = _blocks(raw, n, "IQ3_XXS")
    d, G = _f16(b, 0), grids()["kIQ3XXS"]
    out = np.empty((b.shape[0], 8, 4, 8), np.float32)
    for ib in range(8):
        a = _u32(b, 66 + 4 * ib)
        db = d * (np.float32(0.5) + (a >> 28).astype(np.float32)) * np.float32(0.5)
        for l in range(4):
            g = np.concatenate([G[b[:, 2 + 8 * ib + 2 * l]], G[b[:, 2 + 8 * ib + 2 * l + 1]]], axis=1)
            out[:, ib, l] = db[:, None] * (g.astype(np.float32) * _signs(ksigns((a >> (7 * l)) & 127)))
    return out.reshape(-1)[:n]


def iq3_s_dequant(raw, n):
    """dequantize_row_iq3_s: index qs[8 ib + 2 l] | ((qh[ib] << (8 - 2 l)) & 256) for the first
    entry of group l and qs[8 ib + 2 l + 1] | ((qh[ib] << (7 - 2 l)) & 256) for the second; the
    sign byte signs[4 ib + l]; db = d (1 + 2 * nibble ib of the scale bytes)."""
    b = _blocks(raw, n, "IQ3_S")
    d, G = _f16(b, 0), grids()["kIQ3S"]
    out = np.empty((b.shape[0], 8, 4, 8), np.float32)
    for ib in range(8):
        qh = b[:, 66 + ib]
        db = d * (1 + 2 * ((b[:, 106 + ib // 2] >> (4 * (ib % 2))) & 15)).astype(np.float32)
        for l in range(4):
            i1 = b[:, 2 + 8 * ib + 2 * l] | ((qh << (8 - 2 * l)) & 256)
            i2 = b[:, 2 + 8 * ib + 2 * l + 1] | ((qh << (7 - 2 * l)) & 256)
            g = np.concatenate([G[i1], G[i2]], axis=1)
            out[:, ib, l] = db[:, None] * (g.astype(np.float32) * _signs(b[:, 74 + 4 * ib + l]))
    return out.reshape(-1)[:n]


IQ1_DELTA = np.float32(0.125)


def iq1_s_dequant(raw, n):
    """dequantize_row_iq1_s: qh[ib] (u16) holds 3 high index bits per group (bits 3 l..), a 3-bit
    scale (bits 12-14) and the sign of delta (bit 15); dl = d (2 scale + 1);
    y = dl * (grid[qs[4 ib + l] | high << 8][j] + delta)."""
    b = _blocks(raw, n, "IQ1_S")
    d, G = _f16(b, 0), grids()["kIQ1S"]
    out = np.empty((b.shape[0], 8, 4, 8), np.float32)
    for ib in range(8):
        qh = _u16(b, 34 + 2 * ib)
        dl = d * (2 * ((qh >> 12) & 7) + 1).astype(np.float32)
        delta = np.where(qh & 0x8000, -IQ1_DELTA, IQ1_DELTA).astype(np.float32)
        for l in range(4):
            idx = b[:, 2 + 4 * ib + l] | (((qh >> (3 * l)) & 7) << 8)
            out[:, ib, l] = dl[:, None] * (G[idx].astype(np.float32) + delta[:, None])
    return out.reshape(-1)[:n]


def iq1_m_dequant(raw, n):
    """dequantize_row_iq1_m: no stored d -- its fp16 bits are the top nibbles of the four u16
    scale words; sub-block ib has two 3-bit scales (groups 0-1, 2-3) in scale word ib / 2 at bits
    6 (ib % 2) and + 3; qh[2 ib + l / 2] gives group l its high index bits (<< 8 for even l,
    << 4 for odd l, mask 0x700) and its delta sign (bit 3 for even l, bit 7 for odd l)."""
    b = _blocks(raw, n, "IQ1_M")
    G = grids()["kIQ1S"]
    s = [_u16(b, 48 + 2 * k) for k in range(4)]
    dbits = (s[0] >> 12) | ((s[1] >> 8) & 0xF0) | ((s[2] >> 4) & 0xF00) | (s[3] & 0xF000)
    d = dbits.astype(np.uint16).view(np.float16).astype(np.float32)
    out = np.empty((b.shape[0], 8, 4, 8), np.float32)
    for ib in range(8):
        sw = s[ib // 2] >> (6 * (ib % 2))
        for l in range(4):
            qhb = b[:, 32 + 2 * ib + l // 2]
            idx = b[:, 4 * ib + l] | ((qhb << (4 if l % 2 else 8)) & 0x700)
            neg = qhb & (0x80 if l % 2 else 0x08)
            delta = np.where(neg, -IQ1_DELTA, IQ1_DELTA).astype(np.float32)
            dl = d * (2 * ((sw >> (3 * (l // 2))) & 7) + 1).astype(np.float32)
            out[:, ib, l] = dl[:, None] * (G[idx].astype(np.float32) + delta[:, None])
    return out.reshape(-1)[:n]


def tq1_0_dequant(raw, n):
    """dequantize_row_tq1_0: 48 qs bytes then 4 qh bytes then fp16 d; trit p of a byte is the top
    of (byte * 3^p mod 256) * 3. qs[0:32] gives values 32 p + m (p < 5), qs[32:48] values
    160 + 16 p + m, qh values 240 + 4 p + j (p < 4); y = d (trit - 1)."""
    b = _blocks(raw, n, "TQ1_0")
    d = _f16(b, 52)
    out = np.empty((b.shape[0], 256), np.float32)

    def trit(x, p):
        return ((((x * 3 ** p) & 0xFF) * 3) >> 8).astype(np.float32) - np.float32(1.0)
    for p in range(5):
        out[:, 32 * p:32 * p + 32] = trit(b[:, 0:32], p)
        out[:, 160 + 16 * p:176 + 16 * p] = trit(b[:, 32:48], p)
    for p in range(4):
        out[:, 240 + 4 * p:244 + 4 * p] = trit(b[:, 48:52], p)
    return (out * d[:, None]).reshape(-1)[:n]


def tq2_0_dequant(raw, n):
    """dequantize_row_tq2_0: 64 qs bytes then fp16 d; value 128 g + 32 l + m is bits 2 l of
    qs[32 g + m]; y = d (q - 1)."""
    b = _blocks(raw, n, "TQ2_0")
    d = _f16(b, 64)
    out = np.empty((b.shape[0], 2, 4, 32), np.float32)
    for g in range(2):
        for l in range(4):
            out[:, g, l] = ((b[:, 32 * g:32 * g + 32] >> (2 * l)) & 3).astype(np.float32) - np.float32(1.0)
    return (out.reshape(-1, 256) * d[:, None]).reshape(-1)[:n]


# E2M1 values doubled (ggml's kvalues_mxfp4): codes 0-7 positive, 8-15 their negatives
FP4 = np.array([0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12], np.float32)


def e8m0_half(e):
    """MXFP4's shared exponent halved (the codes are doubled): 2^(e - 128), with the bit
    patterns of the denormals 2^-128 and 2^-127 for e = 0, 1."""
    e = np.asarray(e, np.int64)
    bits = np.where(e < 2, 0x00200000 << e, (e - 1) << 23)
    return bits.astype(np.uint32).view(np.float32)


def ue4m3_half(v):
    """NVFP4's unsigned E4M3 sub-block scale halved: (1 + m/8) 2^(e - 7) / 2, or m 2^-9 / 2 for
    e = 0; the bytes 0 and 0x7F give 0 (bit 7 is not part of the value)."""
    v = np.asarray(v, np.int64)
    e, m = (v >> 3) & 15, (v & 7)
    val = np.where(e == 0, np.ldexp(m.astype(np.float64), -10), np.ldexp((8 + m).astype(np.float64), e - 11))
    return np.where((v == 0) | (v == 0x7F), 0.0, val).astype(np.float32)


def mxfp4_dequant(raw, n):
    """dequantize_row_mxfp4: E8M0 exponent byte then 16 code bytes; value j < 16 is the low
    nibble of byte 1 + j, value 16 + j the high one; y = fp4[q] * e8m0_half(e)."""
    b = _blocks(raw, n, "MXFP4")
    q = b[:, 1:17]
    v = np.concatenate([FP4[q & 15], FP4[q >> 4]], axis=1)
    return (v * e8m0_half(b[:, 0])[:, None]).reshape(-1)[:n]


def nvfp4_dequant(raw, n):
    """dequantize_row_nvfp4: four UE4M3 scale bytes, then 8 code bytes per 16-value sub-block s
    (value 16 s + j: low nibble of byte 4 + 8 s + j for j < 8, high nibble of byte j - 8)."""
    b = _blocks(raw, n, "NVFP4")
    out = np.empty((b.shape[0], 4, 16), np.float32)
    for s in range(4):
        q = b[:, 4 + 8 * s:12 + 8 * s]
        out[:, s] = np.concatenate([FP4[q & 15], FP4[q >> 4]], axis=1) * ue4m3_half(b[:, s])[:, None]
    return out.reshape(-1)[:n]


def q1_0_dequant(raw, n):
    """128 values / 18 bytes: fp16 d, then bit j % 8 of byte 2 + j / 8 selects +d (set) or -d."""
    b = _blocks(raw, n, "Q1_0")
    d = _f16(b, 0)[:, None]
    bits = (b[:, 2:18, None] >> np.arange(8)) & 1
    return np.where(bits.reshape(-1, 128) != 0, d, -d).astype(np.float32).reshape(-1)[:n]


def q2_0_dequant(raw, n):
    """64 values / 18 bytes: fp16 d, then bits 2 (j % 4) of byte 2 + j / 4; y = d (q - 1)."""
    b = _blocks(raw, n, "Q2_0")
    d = _f16(b, 0)[:, None]
    q = (b[:, 2:18, None] >> (2 * np.arange(4))) & 3
    return ((q.reshape(-1, 64).astype(np.float32) - np.float32(1.0)) * d).reshape(-1)[:n]


def f32_dequant(raw, n):
    return _u8(raw)[:4 * n].view(np.float32).copy()


def f16_dequant(raw, n):
    return _u8(raw)[:2 * n].view(np.float16).astype(np.float32)


def bf16_dequant(raw, n):
    return (_u8(raw)[:2 * n].view(np.uint16).astype(np.uint32) << 16).view(np.float32)


DEQUANT = {"IQ2_XXS": iq2_xxs_dequant, "IQ2_XS": iq2_xs_dequant, "IQ2_S": iq2_s_dequant,
           "IQ3_XXS": iq3_xxs_dequant, "IQ3_S": iq3_s_dequant, "IQ1_S": iq1_s_dequant, "IQ1_M": iq1_m_dequant,
           "TQ1_0": tq1_0_dequant, "TQ2_0": tq2_0_dequant, "MXFP4": mxfp4_dequant, "NVFP4": nvfp4_dequant,
           "Q1_0": q1_0_dequant, "Q2_0": q2_0_dequant, "F32": f32_dequant, "F16": f16_dequant,
           "BF16": bf16_dequant}
