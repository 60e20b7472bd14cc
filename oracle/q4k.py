"""GGUF Q4_K oracle (test infrastructure only; see `oracle/__init__.py`).

Follows `ggufload.dequant` for Q4_K (`webtorch/ggufload.py:116-130, 188-202`) and the
`UnquantizedLinear` float32 matmul (`webtorch/_core.py:4462-4481`) that the reference uses for
a dequantized GGUF weight on the CPU.

Pins (tests/test_oracle_q4k.py): a scalar restatement of llama.cpp's published
`dequantize_row_q4_K` loop (the same formula, independent index arithmetic), special cases
(d = dmin = 0 gives zeros; all sub-scales 0 gives -dmin*m; a block with one nonzero code), the
packer round trip (`webpytorch_amd.synth.pack_q4k_scales`) and a brute-force matmul.
"""
import numpy as np

BLOCK_VALS = 256
BLOCK_BYTES = 144


def f16_field(b):
    """(n, 2) uint8 little-endian halves -> (n, 1) float32."""
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32)


def scale_min_k4(s):
    """12 packed bytes per block -> (sc, m), each (n, 8) float32 six-bit values."""
    s = np.asarray(s, np.uint8)
    sc = np.empty((s.shape[0], 8), np.float32)
    m = np.empty((s.shape[0], 8), np.float32)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def q4k_dequant(raw, n):
    """Dequantize the first n values of a Q4_K byte stream to float32.

    Sub-block j (32 values) uses d*sc[j] and dmin*m[j]; byte i of the 32-byte quant group
    q = j // 2 holds value i of sub-block 2q in its low nibble and of 2q+1 in its high
    nibble. Each value is (d*sc) * code - (dmin*m), both products exact in float32."""
    u8 = np.frombuffer(np.ascontiguousarray(raw).tobytes() if not isinstance(raw, bytes) else raw,
                       np.uint8)
    nb = n // BLOCK_VALS
    b = u8[:nb * BLOCK_BYTES].reshape(nb, BLOCK_BYTES)
    d, dmin = f16_field(b[:, 0:2]), f16_field(b[:, 2:4])
    sc, m = scale_min_k4(b[:, 4:16])
    qs = b[:, 16:144]
    out = np.empty((nb, BLOCK_VALS), np.float32)
    for q in range(4):
        grp = qs[:, 32 * q:32 * (q + 1)]
        for half, codes in ((0, grp & 15), (1, grp >> 4)):
            j = 2 * q + half
            scale = d * sc[:, j:j + 1]
            mn = dmin * m[:, j:j + 1]
            out[:, 32 * j:32 * (j + 1)] = scale * codes.astype(np.float32) - mn
    return out.reshape(-1)[:n]


def q4k_matmul(x, rows_bytes, K, N):
    """x (M, K) @ dequant(W).T, W being N rows of K/256 super-blocks -> (M, N) float32."""
    W = q4k_dequant(np.asarray(rows_bytes, np.uint8).reshape(-1), N * K).reshape(N, K)
    return np.asarray(x, np.float32) @ W.T
