"""GPU parity: Q4_K dequant (bit-exact) and GEMV (tolerance) against the oracle."""
import numpy as np
import pytest

from oracle import q4k
from webpytorch_amd import synth

pytestmark = pytest.mark.gpu


def _rel(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max() / (np.abs(ref).max() + 1e-30))


def test_dequant_bit_exact(gpu):
    from webpytorch_amd import core
    W = synth.q4k_layer(1, 4096, 512)
    lin = core.GGMLLinear(W.tobytes(), "Q4_K", 4096, 512)
    got = lin.dequantize().cpu().numpy()
    ref = q4k.q4k_dequant(W.reshape(-1), 512 * 4096).reshape(512, 4096)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_random_bytes_bit_exact(gpu):
    # like the reference's self-check: arbitrary bytes with finite fp16 fields
    import torch
    from webpytorch_amd import core
    raw = np.random.default_rng(0).integers(0, 256, (64, 144), dtype=np.uint8)
    raw[:, 1] &= 0x3B
    raw[:, 3] &= 0x3B
    got = core.q4k_dequant(core.to_device(raw.reshape(-1)), 64).cpu().numpy()
    ref = q4k.q4k_dequant(raw.reshape(-1), 64 * 256)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("M", [1, 2, 3])
def test_config1_gemv(gpu, M):
    """Q4_K GEMV at the Llama-3-8B up_proj shape: x (M, 4096) fp16 -> y (M, 14336) fp32."""
    import torch
    from webpytorch_amd import core
    K, N = 4096, 14336
    W = synth.q4k_layer(0, K, N)
    x = synth.activations(0, M, K, np.float16)
    lin = core.GGMLLinear(W, "Q4_K", K, N)
    got = lin(torch.from_numpy(x)).cpu().numpy()
    assert got.dtype == np.float32 and got.shape == (M, N)
    ref = q4k.q4k_matmul(x, W, K, N)
    assert _rel(got, ref) < 1e-5
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))


# (512, 8000): a width where the kernel walks 8 rows a wave (7 elsewhere)
@pytest.mark.parametrize("K,N", [(256, 2), (768, 33), (8192, 70), (512, 8000)])
def test_gemv_ragged_shapes_and_bias(gpu, K, N):
    import torch
    from webpytorch_amd import core
    W = synth.q4k_layer(K + N, K, N)
    x = synth.activations(K, 1, K, np.float32)
    b = np.linspace(-1, 1, N).astype(np.float32)
    lin = core.GGMLLinear(W, "Q4_K", K, N, bias=b)
    got = lin(torch.from_numpy(x)).cpu().numpy()
    ref = q4k.q4k_matmul(x, W, K, N) + b
    assert _rel(got, ref) < 1e-5


def test_unsupported_type_raises(gpu):
    from webpytorch_amd import core
    assert core.ggml_native_supported("Q4_K") and core.ggml_native_supported("Q5_K")
    assert not core.ggml_native_supported("Q8_K")  # the K-quants' activation type, never a weight's
    with pytest.raises(NotImplementedError):
        core.GGMLLinear(b"\0" * 292, "Q8_K", 256, 1)
    from webpytorch_amd import _lib
    with pytest.raises(NotImplementedError):  # the C ABI refuses an id it has no decoder for
        _lib.call("miq_ggml_dequant_f32", None, 15, None, 1, None)


# ---- Q8_0 and Q6_K (the other types of a Q4_K_M file) ------------------------------------

def _ggml_case(type_name, K, N, seed):
    from oracle import ggml
    W = (synth.q8_0_layer if type_name == "Q8_0" else synth.q6k_layer)(seed, K, N)
    return W, lambda x: ggml.ggml_matmul(x, W, type_name, K, N)


@pytest.mark.parametrize("type_name", ["Q8_0", "Q6_K"])
@pytest.mark.parametrize("M", [1, 3])
def test_q8_0_q6k_gemv_llama3_up_shape(gpu, type_name, M):
    import torch
    from webpytorch_amd import core
    K, N = 4096, 14336
    W, ref_fn = _ggml_case(type_name, K, N, 3)
    x = synth.activations(3, M, K, np.float16)
    got = core.GGMLLinear(W, type_name, K, N)(torch.from_numpy(x)).cpu().numpy()
    ref = ref_fn(x)
    assert got.shape == (M, N) and _rel(got, ref) < 1e-5
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))


@pytest.mark.parametrize("type_name,K,N", [("Q8_0", 32, 2), ("Q8_0", 96, 33), ("Q8_0", 8192, 70),
                                           ("Q6_K", 256, 2), ("Q6_K", 768, 33), ("Q6_K", 8192, 70)])
def test_q8_0_q6k_ragged_rows_bias_dtypes(gpu, type_name, K, N):
    """Odd block counts per row put every other row at a 2-byte offset; fp32 and fp16
    activations, fp16 output, bias."""
    import torch
    from webpytorch_amd import core
    W, ref_fn = _ggml_case(type_name, K, N, K + N)
    b = np.linspace(-1, 1, N).astype(np.float32)
    lin = core.GGMLLinear(W, type_name, K, N, bias=b)
    for xdt in (np.float32, np.float16):
        x = synth.activations(K, 2, K, xdt)
        ref = ref_fn(x) + b
        got = lin(torch.from_numpy(x)).cpu().numpy()
        assert _rel(got, ref) < 1e-5
        got16 = lin.forward(torch.from_numpy(x), out_dtype=torch.float16).cpu().numpy()
        assert got16.dtype == np.float16
        assert np.all(np.abs(got16.astype(np.float32) - ref) <= 1e-3 + 1e-2 * np.abs(ref))


@pytest.mark.parametrize("type_name,K,N", [("Q8_0", 96, 33), ("Q6_K", 768, 33), ("Q4_K", 768, 33)])
def test_dequantize_every_native_type_bit_exact(gpu, type_name, K, N):
    """GGMLLinear.dequantize decodes the layer's own type (the reference's `ggufload.dequant`),
    including rows at 2-byte offsets."""
    from oracle import ggml
    from webpytorch_amd import core
    W = {"Q8_0": synth.q8_0_layer, "Q6_K": synth.q6k_layer, "Q4_K": synth.q4k_layer}[type_name](7, K, N)
    got = core.GGMLLinear(W, type_name, K, N).dequantize().cpu().numpy()
    if type_name == "Q4_K":
        ref = q4k.q4k_dequant(W.reshape(-1), N * K).reshape(N, K)
    else:
        ref = ggml.DEQUANT[type_name][0](W.reshape(-1), N * K).reshape(N, K)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("type_name,K,N", [("Q4_K", 1024, 40), ("Q6_K", 512, 33), ("Q8_0", 128, 17)])
def test_ggml_matmul_accepts_the_reference_transposed_layout(gpu, type_name, K, N):
    """`ggml_matmul` given the reference's (word, row) u32 layout (`ggml_transpose`,
    `webtorch/_core.py:4315-4344`: word w of row r at w * N + r, the row's tail bytes
    zero-padded to a word) gives the same result as the native rows."""
    import torch
    from webpytorch_amd import core
    W = {"Q8_0": synth.q8_0_layer, "Q6_K": synth.q6k_layer, "Q4_K": synth.q4k_layer}[type_name](9, K, N)
    rows = np.asarray(W, np.uint8).reshape(N, -1)
    rowb = rows.shape[1]
    nw = (rowb + 3) // 4
    padded = np.zeros((N, nw * 4), np.uint8)
    padded[:, :rowb] = rows
    transposed = np.ascontiguousarray(padded.view(np.uint32).reshape(N, nw).T).reshape(-1)
    x = torch.from_numpy(synth.activations(9, 2, K, np.float32)).cuda()
    a = core.ggml_matmul(x, core.ggml_transpose(rows, N, rowb), type_name, K, N).cpu().numpy()
    b = core.ggml_matmul(x, torch.from_numpy(transposed.view(np.int32)).cuda(), type_name, K, N).cpu().numpy()
    assert np.array_equal(a, b)
    with pytest.raises(ValueError):
        core.ggml_matmul(x, torch.from_numpy(transposed.view(np.int32)[:-1]).cuda(), type_name, K, N)


# ---- the other llama.cpp block types -------------------------------------------------------

NEW_TYPES = ["Q4_0", "Q4_1", "Q5_0", "Q5_1", "IQ4_NL", "IQ4_XS", "Q5_K", "Q2_K", "Q3_K"]


@pytest.mark.parametrize("type_name", NEW_TYPES)
def test_new_type_dequant_bit_exact_random_blocks(gpu, type_name):
    """Device dequant of random blocks (every code and sub-scale byte uniform, fp16 fields of
    mixed sign and magnitude, subnormals included, kept finite) matches the oracle bit for
    bit."""
    import torch
    from oracle import ggml
    from webpytorch_amd import core
    f, vals, nbytes = ggml.DEQUANT[type_name]
    g = np.random.default_rng(vals * 1000 + nbytes)
    nb = 1531
    raw = g.integers(0, 256, (nb, nbytes), dtype=np.uint8)
    for off in ggml.F16_FIELDS[type_name]:
        h = (g.standard_normal(nb) * np.exp2(g.integers(-26, 6, nb))).astype(np.float16)
        raw[:, off:off + 2] = h.view(np.uint8).reshape(nb, 2)
    got = core.ggml_dequant(torch.from_numpy(raw.reshape(-1)).cuda(), type_name, nb).cpu().numpy()
    ref = f(raw.reshape(-1), nb * vals)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("type_name", NEW_TYPES)
@pytest.mark.parametrize("M", [1, 2, 5])
def test_new_type_gemv_llama3_up_shape(gpu, type_name, M):
    """The llama-3-8B up projection (4096 -> 14336) in each type against the oracle's dequant
    times x, one to five activation rows."""
    import torch
    from oracle import ggml
    from webpytorch_amd import core
    K, N = 4096, 14336
    W = synth.ggml_layer(type_name, 3, K, N)
    x = synth.activations(3, M, K, np.float16)
    got = core.GGMLLinear(W, type_name, K, N)(torch.from_numpy(x)).cpu().numpy()
    ref = ggml.ggml_matmul(x, W, type_name, K, N)
    assert got.shape == (M, N) and _rel(got, ref) < 1e-5
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))


@pytest.mark.parametrize("type_name", NEW_TYPES)
def test_new_type_ragged_rows_bias_dtypes(gpu, type_name):
    """Odd block counts per row (rows at 2-byte offsets), a ragged row count, bias, fp32 and
    fp16 activations, fp16 output, and GGMLLinear.dequantize bit-exact."""
    import torch
    from oracle import ggml
    from webpytorch_amd import core
    vals = ggml.DEQUANT[type_name][1]
    K, N = 3 * vals if vals == 256 else 7 * vals, 37
    W = synth.ggml_layer(type_name, K + N, K, N)
    b = np.linspace(-1, 1, N).astype(np.float32)
    lin = core.GGMLLinear(W, type_name, K, N, bias=b)
    for xdt in (np.float32, np.float16):
        x = synth.activations(K, 2, K, xdt)
        ref = ggml.ggml_matmul(x, W, type_name, K, N) + b
        got = lin(torch.from_numpy(x)).cpu().numpy()
        assert _rel(got, ref) < 1e-5
        got16 = lin.forward(torch.from_numpy(x), out_dtype=torch.float16).cpu().numpy()
        assert got16.dtype == np.float16
        assert np.all(np.abs(got16.astype(np.float32) - ref) <= 1e-3 + 1e-2 * np.abs(ref))
    deq = lin.dequantize().cpu().numpy()
    ref = ggml.DEQUANT[type_name][0](W.reshape(-1), N * K).reshape(N, K)
    assert np.array_equal(deq.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("type_name", NEW_TYPES)
def test_new_type_prefill_rows(gpu, type_name):
    """More activation rows than the one-row kernels take (a prefill of 24 tokens) go through
    the same layer and match the oracle."""
    import torch
    from oracle import ggml
    from webpytorch_amd import core
    K, N = 2048, 96
    W = synth.ggml_layer(type_name, 11, K, N)
    x = synth.activations(11, 24, K, np.float32)
    got = core.GGMLLinear(W, type_name, K, N)(torch.from_numpy(x)).cpu().numpy()
    ref = ggml.ggml_matmul(x, W, type_name, K, N)
    assert _rel(got, ref) < 1e-5
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))


# ---- Q4_K prefill rows on the matrix cores ------------------------------------------------

@pytest.mark.parametrize("M,K,N", [(9, 256, 64), (100, 768, 70), (64, 4096, 14336), (300, 2048, 512),
                                   (520, 256, 7200)])
@pytest.mark.parametrize("xdt", [np.float32, np.float16])
def test_q4k_gemm_prefill_rows(gpu, M, K, N, xdt):
    """Rows above the GEMV's take the matrix-core GEMM (exact sub-block decomposition); against
    the oracle's dequant times x at row-tile and column-tile tails, with bias and fp16 output.
    (520, 256, 7200) has grid enough for two 16-column groups per wave (9 x 57 tiles)."""
    import torch
    from webpytorch_amd import core
    W = synth.q4k_layer(M + K, K, N)
    b = np.linspace(-1, 1, N).astype(np.float32)
    lin = core.GGMLLinear(W, "Q4_K", K, N, bias=b)
    x = synth.activations(M, M, K, xdt)
    ref = q4k.q4k_matmul(x.astype(np.float32), W, K, N) + b
    got = lin(torch.from_numpy(x)).cpu().numpy()
    assert _rel(got, ref) < 1e-5
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))
    got16 = lin.forward(torch.from_numpy(x), out_dtype=torch.float16).cpu().numpy()
    assert np.all(np.abs(got16.astype(np.float32) - ref) <= 1e-3 + 1e-2 * np.abs(ref))
    assert np.array_equal(lin(torch.from_numpy(x)).cpu().numpy(), got)  # deterministic


def test_q4k_gemm_row_scales_and_nonfinite(gpu):
    """fp32 rows of very different magnitude keep their relative accuracy (each row is split
    at its own scale); a row holding NaN gives NaN and an Inf row gives non-finite outputs,
    while the other rows are unaffected."""
    import torch
    from webpytorch_amd import core
    K, N, M = 1024, 192, 24
    W = synth.q4k_layer(5, K, N)
    lin = core.GGMLLinear(W, "Q4_K", K, N)
    x = synth.activations(5, M, K, np.float32)
    x *= np.logspace(-6, 6, M, dtype=np.float32)[:, None]
    ref = q4k.q4k_matmul(x, W, K, N)
    got = lin(torch.from_numpy(x)).cpu().numpy()
    for m in range(M):
        assert np.abs(got[m] - ref[m]).max() <= 1e-5 * np.abs(ref[m]).max(), m
    x[3, 7] = np.nan
    x[5, 9] = np.inf
    got = lin(torch.from_numpy(x)).cpu().numpy()
    assert np.isnan(got[3]).all() and not np.isfinite(got[5]).any()
    keep = [m for m in range(M) if m not in (3, 5)]
    assert np.abs(got[keep] - ref[keep]).max() <= 1e-5 * np.abs(ref[keep]).max()


# ---- Q5_K / Q6_K / Q8_0 prefill rows on the matrix cores -----------------------------------

KQ_GEMM_CASES = [(9, 256, 64, np.float32), (100, 768, 70, np.float16), (100, 768, 70, np.float32),
                 (33, 1280, 1000, np.float32), (520, 256, 7200, np.float16), (64, 4096, 14336, np.float16),
                 (300, 2048, 512, np.float32)]


@pytest.mark.parametrize("type_name", ["Q5_K", "Q6_K", "Q8_0"])
@pytest.mark.parametrize("M,K,N,xdt", KQ_GEMM_CASES)
def test_kquant_gemm_prefill_rows(gpu, type_name, M, K, N, xdt):
    """Rows above the GEMV's take `miq_ggml_gemm`: against the oracle's exact dequant times x,
    at row- and column-tile tails, with bias and fp16 output. K = 768 and 1280 give rows of an odd
    number of super-blocks, so Q6_K's 210-byte blocks start at both 2-byte residues; (520, 256,
    7200) takes two 16-column groups per wave. Block bytes are uniform random: Q6_K scales cover
    -128..127 and codes 0..63, Q8_0 codes -128..127."""
    import torch
    from oracle import ggml
    from webpytorch_amd import core
    assert core._ggml_gemm_taken(type_name, M, K)
    W = synth.ggml_layer(type_name, M + K + N, K, N)
    b = np.linspace(-1, 1, N).astype(np.float32)
    lin = core.GGMLLinear(W, type_name, K, N, bias=b)
    x = synth.activations(M + 1, M, K, xdt)
    ref = ggml.ggml_matmul(x.astype(np.float32), W, type_name, K, N) + b
    got = lin(torch.from_numpy(x)).cpu().numpy()
    assert _rel(got, ref) < 1e-5
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))
    got16 = lin.forward(torch.from_numpy(x), out_dtype=torch.float16).cpu().numpy()
    assert np.all(np.abs(got16.astype(np.float32) - ref) <= 1e-3 + 1e-2 * np.abs(ref))
    assert np.array_equal(lin(torch.from_numpy(x)).cpu().numpy(), got)  # deterministic


@pytest.mark.parametrize("type_name", ["Q5_K", "Q6_K", "Q8_0"])
def test_kquant_gemm_extreme_codes_and_row_scales(gpu, type_name):
    """Every code and scale at its extreme (Q6_K: codes 0 and 63, scales -128 and 127; Q8_0:
    codes -128 and 127; Q5_K: codes 31 with 6-bit scales 63), fp32 rows of very different
    magnitude, and NaN / Inf rows that leave the other rows alone."""
    import torch
    from oracle import ggml
    from webpytorch_amd import core
    K, N, M = 1024, 96, 24
    W = synth.ggml_layer(type_name, 9, K, N).reshape(-1, ggml.DEQUANT[type_name][2]).copy()
    g = np.random.default_rng(9)
    if type_name == "Q6_K":
        W[:, 0:192] = g.choice(np.array([0x00, 0xFF], np.uint8), W[:, 0:192].shape)
        W[:, 192:208] = g.choice(np.array([0x80, 0x7F], np.uint8), W[:, 192:208].shape)
    elif type_name == "Q8_0":
        W[:, 2:34] = g.choice(np.array([0x80, 0x7F], np.uint8), W[:, 2:34].shape)
    else:
        W[:, 4:176] = 0xFF
    W = W.reshape(-1)
    lin = core.GGMLLinear(W, type_name, K, N)
    x = synth.activations(5, M, K, np.float32)
    x *= np.logspace(-6, 6, M, dtype=np.float32)[:, None]
    ref = ggml.ggml_matmul(x, W, type_name, K, N)
    got = lin(torch.from_numpy(x)).cpu().numpy()
    for m in range(M):
        assert np.abs(got[m] - ref[m]).max() <= 1e-5 * np.abs(ref[m]).max(), m
    x[3, 7] = np.nan
    x[5, 9] = np.inf
    got = lin(torch.from_numpy(x)).cpu().numpy()
    assert np.isnan(got[3]).all() and not np.isfinite(got[5]).any()
    keep = [m for m in range(M) if m not in (3, 5)]
    for m in keep:
        assert np.abs(got[m] - ref[m]).max() <= 1e-5 * np.abs(ref[m]).max(), m
