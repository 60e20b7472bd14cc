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


@pytest.mark.parametrize("K,N", [(256, 2), (768, 33), (8192, 70)])
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
    assert core.ggml_native_supported("Q4_K") and not core.ggml_native_supported("Q6_K")
    with pytest.raises(NotImplementedError):
        core.GGMLLinear(b"\0" * 210, "Q6_K", 256, 1)
