"""GGUF Q8_0 and Q6_K oracle (test infrastructure only; see `oracle/__init__.py`).

Follows `ggufload.dequant` for Q8_0 (`webtorch/ggufload.py:140-145`) and Q6_K
(`webtorch/ggufload.py:203-222`), and the `UnquantizedLinear` float32 matmul
(`webtorch/_core.py:4462-4481`) that the reference uses for a dequantized GGUF weight on the CPU.
Both dequantizations are exact in float32: d (fp16, 11 significant bits) times an int8 code or
scale (8 bits) times a 6-bit code stays within float32's 24 bits, so the order of the products
does not matter.

Pins (tests/test_oracle_ggml.py): a scalar, per-element restatement of llama.cpp's published
`dequantize_row_q8_0` / `dequantize_row_q6_K` loops (index arithmetic written independently of
the vectorized form below); special cases (d = 0 gives zeros; d = 1 and unit scales give the
raw codes, minus 32 for Q6_K; one nonzero byte moves exactly the weights that byte feeds); the
matmul against a float64 brute force.
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


DEQUANT = {"Q8_0": (q8_0_dequant, Q8_0_VALS, Q8_0_BYTES), "Q6_K": (q6k_dequant, Q6K_VALS, Q6K_BYTES)}


def ggml_matmul(x, rows_bytes, type_name, K, N):
    """x (M, K) @ dequant(W).T -> (M, N) float32, W being N rows of K / block-values blocks."""
    f, vals, nbytes = DEQUANT[type_name]
    W = f(np.asarray(rows_bytes, np.uint8).reshape(-1), N * K).reshape(N, K)
    return np.asarray(x, np.float32) @ W.T
