"""The oracle for the GGUF types beyond the K-quants (i-quant grids, ternary, fp4, 1/2-bit,
unquantized matrices) against the reference's own `ggufload.dequant` output on random blocks
(`tests/golden/ggml_ext.npz`, written by `tests/golden/make_golden.py` in the build container),
the codebook tables against the reference's (SHA-256 of their values), and special cases that
fix each field's role independently of the vectorized restatement: zero scales, a unit scale
that exposes the raw codebook entry, one sign / index / high bit moving exactly the values it
feeds."""
import hashlib
import os

import numpy as np
import pytest

from oracle import ggml, ggml_ext

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ggml_ext.npz")

# SHA-256 of each codebook's values (int8 per value, entries in order), taken from the reference's
# `webtorch/iqtables.py` by `webpytorch_amd/csrc/gen_iq_grids.py`
DIGESTS = {"kIQ2XXS": "05826b5d3e472a3a78f196be62ac78acf81df0f909626e12ab9fa2a5d490dd54",
           "kIQ2XS": "06e47aaca60b4dc1d9b5a3f34540437058a6b142b4d7a59d5ded769b4d1bf1de",
           "kIQ2S": "e1aa1473412b0552c2174c30ef22ab4073f6a181b85a17056e8249bd2932fd88",
           "kIQ3XXS": "46e35f5a997efdee6c99ce57854c8a0d4f0ff8ca57e5e8a60c0793ea580acf5d",
           "kIQ3S": "bd1af4945a1717c65610b0284e4628b9a1ba3b306fae3a06f6e5f597356e349f",
           "kIQ1S": "07540ffc1aeaf6ad4d97e96b0fcc765aae39671d4ae4a27bbd0e796fde167c6a"}


def _cases():
    z = np.load(GOLDEN)
    n = len({k.split(".")[0] for k in z.files})
    return [(str(z["c%02d.type" % i]), z["c%02d.raw" % i], z["c%02d.y" % i]) for i in range(n)]


def test_fixture_covers_every_type():
    assert {c[0] for c in _cases()} == set(ggml_ext.DEQUANT)


@pytest.mark.parametrize("case", range(len(_cases())))
def test_oracle_matches_reference_dequant(case):
    name, raw, want = _cases()[case]
    vals, nbytes = ggml_ext.BLOCKS[name]
    n = want.size
    got = ggml.DEQUANT[name][0](raw, n)
    assert got.dtype == np.float32 and got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), name


def test_codebook_tables_match_the_reference():
    g = ggml_ext.grids()
    sizes = {"kIQ2XXS": (256, 8), "kIQ2XS": (512, 8), "kIQ2S": (1024, 8), "kIQ3XXS": (256, 4), "kIQ3S": (512, 4),
             "kIQ1S": (2048, 8)}
    for name, shape in sizes.items():
        v = np.ascontiguousarray(g[name].astype(np.int8))
        assert v.shape == shape
        assert hashlib.sha256(v.tobytes()).hexdigest() == DIGESTS[name], name
    # the value sets the formats use
    assert set(np.unique(g["kIQ2XXS"])) | set(np.unique(g["kIQ2XS"])) | set(np.unique(g["kIQ2S"])) == {8, 25, 43}
    assert set(np.unique(g["kIQ3XXS"])) <= set(range(4, 63, 8)) | {62}
    assert set(np.unique(g["kIQ1S"])) == {-1, 0, 1}
    for name in sizes:  # a codebook has no repeated entry
        assert len({tuple(r) for r in g[name]}) == sizes[name][0], name


def test_ksigns_parity_rule():
    s = np.arange(128)
    k = ggml_ext.ksigns(s)
    assert np.all(k & 127 == s)
    assert np.all(np.array([bin(int(v)).count("1") for v in k]) % 2 == 0)  # even parity over 8 bits
    assert k[1] == 0x81 and k[3] == 0x03 and k[127] == 0xFF


def _block(name, fill=0):
    vals, nbytes = ggml_ext.BLOCKS[name]
    return np.full(nbytes, fill, np.uint8)


def _set_f16(b, off, v):
    b[off:off + 2] = np.array([v], np.float16).view(np.uint8)


@pytest.mark.parametrize("name", ["IQ2_XXS", "IQ2_XS", "IQ2_S", "IQ3_XXS", "IQ3_S", "IQ1_S", "TQ1_0", "TQ2_0",
                                  "Q1_0", "Q2_0"])
def test_zero_scale_gives_zeros(name):
    g = np.random.default_rng(1)
    b = g.integers(0, 256, ggml_ext.BLOCKS[name][1], dtype=np.uint8)
    for off in ggml_ext.F16_FIELDS[name]:
        _set_f16(b, off, 0.0)
    assert np.all(ggml.DEQUANT[name][0](b, ggml_ext.BLOCKS[name][0]) == 0)


def test_iq2_xxs_fields():
    """d = 8 and scale 0 make db = 8 * 0.5 / 4 = 1, so values are grid entries with signs."""
    G = ggml_ext.grids()["kIQ2XXS"]
    b = _block("IQ2_XXS")
    _set_f16(b, 0, 8.0)
    # sub-block 3: grid indices 5, 17, 200, 255; sign index of group 2 = 1 (ksigns 0x81: values 0, 7)
    b[2 + 8 * 3:6 + 8 * 3] = [5, 17, 200, 255]
    b[6 + 8 * 3:10 + 8 * 3] = np.array([1 << 14], np.uint32).view(np.uint8)
    y = ggml.DEQUANT["IQ2_XXS"][0](b, 256).reshape(8, 4, 8)
    assert np.array_equal(y[3, 0], G[5]) and np.array_equal(y[3, 1], G[17]) and np.array_equal(y[3, 3], G[255])
    want = G[200].astype(np.float32)
    want[[0, 7]] *= -1
    assert np.array_equal(y[3, 2], want)
    assert np.all(y[[0, 1, 2, 4, 5, 6, 7]] == np.broadcast_to(G[0], (7, 4, 8)))  # index 0 elsewhere
    # the 4-bit scale: 15 gives d (0.5 + 15) / 4 = 31 times the scale-0 value
    b[6 + 8 * 3 + 3] |= 0xF0
    y2 = ggml.DEQUANT["IQ2_XXS"][0](b, 256).reshape(8, 4, 8)
    assert np.array_equal(y2[3], y[3] * np.float32(31))


def test_iq3_s_high_bits_and_signs():
    """IQ3_S: qh bit 2l (8 - 2l shift) lifts the first entry of group l past 256, bit 2l + 1 the
    second; the sign byte is a plain mask; scale nibble s gives d (1 + 2 s)."""
    G = ggml_ext.grids()["kIQ3S"]
    b = _block("IQ3_S")
    _set_f16(b, 0, 1.0)
    b[66 + 2] = 0b00000100  # sub-block 2, group 1, first entry
    b[74 + 4 * 2 + 1] = 0b10000001  # sub-block 2, group 1: values 0 and 7 negated
    b[106 + 1] = 0x30  # sub-block 3's nibble (high of byte 1) = 3 -> d * 7
    y = ggml.DEQUANT["IQ3_S"][0](b, 256).reshape(8, 4, 8)
    first = G[256].astype(np.float32)
    want = np.concatenate([first, G[0].astype(np.float32)])
    want[[0, 7]] *= -1
    assert np.array_equal(y[2, 1], want)
    assert np.array_equal(y[3, 0], np.tile(G[0], 2).astype(np.float32) * 7)


def test_iq1_s_and_m_offsets():
    """IQ1_S: value d (2 s + 1) (grid + delta), delta = -1/8 when qh bit 15 is set, else +1/8.
    IQ1_M: d is spread over the scale words' top nibbles; groups 0-1 take the low 3-bit scale."""
    G = ggml_ext.grids()["kIQ1S"]
    b = _block("IQ1_S")
    _set_f16(b, 0, 2.0)
    b[2 + 4 * 5 + 2] = 7  # sub-block 5, group 2: index 7
    b[34 + 2 * 5:36 + 2 * 5] = np.array([(1 << 15) | (3 << 12)], np.uint16).view(np.uint8)
    y = ggml.DEQUANT["IQ1_S"][0](b, 256).reshape(8, 4, 8)
    assert np.array_equal(y[5, 2], (G[7] - 0.125).astype(np.float32) * 14)
    assert np.array_equal(y[5, 0], (G[0] - 0.125).astype(np.float32) * 14)
    assert np.array_equal(y[0, 0], (G[0] + 0.125).astype(np.float32) * 2)
    m = _block("IQ1_M")
    d = np.array([4.0], np.float16).view(np.uint16)[0]
    sw = np.zeros(4, np.uint16)
    for k in range(4):
        sw[k] = ((int(d) >> (4 * k)) & 15) << 12
    sw[0] |= (1 << 3)  # sub-block 0: high scale 1 (groups 2-3: 4 * 3)
    m[48:56] = sw.view(np.uint8)
    m[32] = 0x08  # sub-block 0, group 0: negative delta
    y = ggml.DEQUANT["IQ1_M"][0](m, 256).reshape(8, 4, 8)
    assert np.array_equal(y[0, 0], (G[0] - 0.125).astype(np.float32) * 4)
    assert np.array_equal(y[0, 1], (G[0] + 0.125).astype(np.float32) * 4)
    assert np.array_equal(y[0, 2], (G[0] + 0.125).astype(np.float32) * 12)


def test_ternary_and_low_bit_layouts():
    """TQ2_0 value 128 g + 32 l + m is bits 2 l of byte 32 g + m; TQ1_0's trits are base-3 digits
    (a byte of 3^5 * t / 243 rounded up holds t in its first trit); Q1_0 / Q2_0 bit order."""
    b = _block("TQ2_0")
    _set_f16(b, 64, 1.0)
    b[32 + 5] = 0b10 << 4  # g 1, m 5, l 2 -> 2 - 1 = +1 at 128 + 64 + 5
    y = ggml.DEQUANT["TQ2_0"][0](b, 256)
    assert y[128 + 64 + 5] == 1.0 and np.sum(y != -1.0) == 1
    t = _block("TQ1_0")
    _set_f16(t, 52, 1.0)
    # digits (most significant first) 2, 0, 1, 1, 0 in a byte: q = ceil(n * 256 / 243)
    n = 2 * 81 + 0 * 27 + 1 * 9 + 1 * 3 + 0
    t[7] = (n * 256 + 242) // 243
    y = ggml.DEQUANT["TQ1_0"][0](t, 256)
    assert [y[32 * p + 7] for p in range(5)] == [1.0, -1.0, 0.0, 0.0, -1.0]
    q1 = _block("Q1_0")
    _set_f16(q1, 0, 0.5)
    q1[2 + 3] = 0b00100001
    y = ggml.DEQUANT["Q1_0"][0](q1, 128)
    assert y[24] == 0.5 and y[29] == 0.5 and np.sum(y == 0.5) == 2 and np.sum(y == -0.5) == 126
    q2 = _block("Q2_0")
    _set_f16(q2, 0, 2.0)
    q2[2 + 4] = 0b11 << 2  # value 17 = byte 4 bits 2-3: 3 - 1 = 2 -> 4
    y = ggml.DEQUANT["Q2_0"][0](q2, 64)
    assert y[17] == 4.0 and np.sum(y != -2.0) == 1


def test_fp4_scales():
    """MXFP4: e8m0 e scales the doubled E2M1 codes by 2^(e - 128); NVFP4: UE4M3 byte (e, m)
    gives (8 + m) 2^(e - 11), m 2^-10 for e = 0, and the bytes 0 and 0x7F give 0."""
    mx = _block("MXFP4")
    mx[0] = 130
    mx[1:17] = np.arange(16, dtype=np.uint8) | (np.arange(16, dtype=np.uint8)[::-1] << 4)
    y = ggml.DEQUANT["MXFP4"][0](mx, 32)
    assert np.array_equal(y[:16], ggml_ext.FP4 * 4) and np.array_equal(y[16:], ggml_ext.FP4[::-1] * 4)
    assert ggml_ext.e8m0_half(0) == np.float32(2.0 ** -128) and ggml_ext.e8m0_half(1) == np.float32(2.0 ** -127)
    assert ggml_ext.e8m0_half(255) == np.float32(2.0 ** 127)
    assert ggml_ext.ue4m3_half(0x7F) == 0 and ggml_ext.ue4m3_half(0) == 0
    assert ggml_ext.ue4m3_half((7 << 3) | 3) == np.float32(11 * 2.0 ** -4)
    assert ggml_ext.ue4m3_half(5) == np.float32(5 * 2.0 ** -10)
    nv = _block("NVFP4")
    nv[0:4] = [(11 << 3), 0, (12 << 3) | 4, 0x7F]  # scales 8, 0, 24, 0
    nv[4:36] = 0x71  # every code pair: low 1 (value 1), high 7 (value 12)
    y = ggml.DEQUANT["NVFP4"][0](nv, 64).reshape(4, 16)
    assert np.all(y[0, :8] == 8) and np.all(y[0, 8:] == 96) and np.all(y[1] == 0) and np.all(y[3] == 0)
    assert np.all(y[2, :8] == 24) and np.all(y[2, 8:] == 288)


def test_dense_types():
    g = np.random.default_rng(3)
    v = g.standard_normal(37).astype(np.float32)
    assert np.array_equal(ggml.DEQUANT["F32"][0](v.tobytes(), 37), v)
    h = v.astype(np.float16)
    assert np.array_equal(ggml.DEQUANT["F16"][0](h.tobytes(), 37), h.astype(np.float32))
    bf = (v.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(ggml.DEQUANT["BF16"][0](bf.tobytes(), 37), (bf.astype(np.uint32) << 16).view(np.float32))


@pytest.mark.parametrize("name", sorted(ggml_ext.DEQUANT))
def test_matmul_brute_force(name):
    from webpytorch_amd import synth
    vals = ggml_ext.BLOCKS[name][0]
    K = 2 * vals if vals > 1 else 40
    W = synth.ggml_layer(name, 5, K, 3, scale=0.01)
    x = np.random.default_rng(5).standard_normal((2, K)).astype(np.float32)
    Wd = ggml.DEQUANT[name][0](W.reshape(-1), 3 * K).reshape(3, K).astype(np.float64)
    ref = x.astype(np.float64) @ Wd.T
    got = ggml.ggml_matmul(x, W, name, K, 3)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6 * np.abs(ref).max())
