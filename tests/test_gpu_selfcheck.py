"""GPU: the first-use known-answer checks (`_ggml_selfcheck`, `webtorch/_core.py:3684-3717`, and
the same for every GPTQ product path) run once per kernel class and device, are skipped under
graph capture, and raise RuntimeError when the kernel disagrees with the exact dequant. The
mismatch is planted on the host side of the check (its float64 reference product is made wrong),
never in a kernel."""
import numpy as np
import pytest

from webpytorch_amd import synth

pytestmark = pytest.mark.gpu


def _fresh(monkeypatch):
    from webpytorch_amd import core
    monkeypatch.setattr(core, "_CHECKED", set())
    return core


@pytest.mark.parametrize("type_name", ["Q4_K", "Q6_K", "Q8_0"])
def test_ggml_check_runs_once_per_mode(gpu, monkeypatch, type_name):
    import torch
    core = _fresh(monkeypatch)
    K, N = 512, 64
    W = {"Q8_0": synth.q8_0_layer, "Q6_K": synth.q6k_layer, "Q4_K": synth.q4k_layer}[type_name](1, K, N)
    lin = core.GGMLLinear(W, type_name, K, N)
    dev = torch.cuda.current_device()
    for M, mode in ((1, 1), (2, 2), (5, 0), (7, 0)):
        lin(torch.from_numpy(synth.activations(1, M, K, np.float32)))
        assert ("ggml", type_name, mode, dev) in core._CHECKED
    assert len([k for k in core._CHECKED if k[0] == "ggml"]) == 3
    lin(torch.from_numpy(synth.activations(1, 24, K, np.float32)))  # prefill rows: the matrix-core GEMM
    assert ("ggml", type_name, -1, dev) in core._CHECKED
    if type_name == "Q8_0":  # K not a multiple of 256: prefill rows take the GEMV row by row
        core._CHECKED.discard(("ggml", type_name, -1, dev))
        lin96 = core.GGMLLinear(synth.q8_0_layer(2, 96, N), "Q8_0", 96, N)
        lin96(torch.from_numpy(synth.activations(2, 24, 96, np.float32)))
        assert ("ggml", type_name, -1, dev) not in core._CHECKED


@pytest.mark.parametrize("M,dt", [(1, "float32"), (4, "float32"), (12, "float16"), (40, "float16"), (1, "float16")])
def test_gptq_check_per_path(gpu, monkeypatch, M, dt):
    import torch
    core = _fresh(monkeypatch)
    L = synth.gptq_layer(2, 512, 256, 128, 4)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 128, 4)
    ql(torch.from_numpy(synth.activations(2, M, 512, getattr(np, dt))))
    keys = [k for k in core._CHECKED if k[0] == "gptq"]
    assert len(keys) == 1 and keys[0][3] == core._gptq_path(M, getattr(torch, dt))


def test_check_raises_on_a_mismatch(gpu, monkeypatch):
    import torch
    core = _fresh(monkeypatch)
    real = core._reference_product
    monkeypatch.setattr(core, "_reference_product", lambda x, W: real(x, W) * 1.01)
    W = synth.q4k_layer(3, 256, 8)
    with pytest.raises(RuntimeError, match="Q4_K.*wrong"):
        core.GGMLLinear(W, "Q4_K", 256, 8)(torch.from_numpy(synth.activations(3, 1, 256, np.float32)))
    L = synth.gptq_layer(3, 256, 64, 128, 8)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 128, 8)
    with pytest.raises(RuntimeError, match="int8.*wrong"):
        ql(torch.from_numpy(synth.activations(3, 1, 256, np.float32)))


def test_no_check_under_graph_capture(gpu, monkeypatch):
    import torch
    core = _fresh(monkeypatch)
    L = synth.gptq_layer(4, 256, 64, 128, 4)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 128, 4)
    x = torch.from_numpy(synth.activations(4, 1, 256, np.float32)).cuda()
    ws = core.workspace(core.gemv_workspace_bytes(1, 256, 64, 128, 4, 0))
    out = torch.empty((1, 64), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        core._gptq_matmul(x, ql.qweight, ql.qzeros, ql.scales, 256, 64, 128, 4, 1.0, bias=ql.bias, out=out, ws=ws)
    assert not core._CHECKED
    g.replay()
    torch.cuda.synchronize()
    ref = ql(x)  # eager: now checked
    assert core._CHECKED
    assert torch.allclose(out, ref, rtol=1e-5, atol=1e-6)


def test_capture_runs_the_one_row_checks_first(gpu, monkeypatch):
    """`CausalLM.capture` runs the one-row check of each product class its step uses before
    capturing (checks are skipped under capture): here fp32-scaled, zero-offset-0 layers (the
    quantize-on-load and tied-head class) and the AutoGPTQ fp16-scaled class."""
    import torch
    from webpytorch_amd import llm
    core = _fresh(monkeypatch)
    w = synth.decoder_weights(3, L=1, H=256, NH=4, NKV=2, HD=64, I=512, V=1024, gs=128, bits=4)
    m = llm.CausalLM.from_weights(w, lmax=32, persistent=False)
    m.capture()
    dev = torch.cuda.current_device()
    keys = {k for k in core._CHECKED if k[0] == "gptq" and k[-1] == dev}
    assert ("gptq", 4, 128, 1, torch.float32, torch.float32, 0.0, dev) in keys   # the tied head
    assert ("gptq", 4, 128, 1, torch.float32, torch.float16, 1.0, dev) in keys   # the layers


def test_quantized_linear_nbytes_is_the_reference_count(gpu):
    """`QuantizedLinear.nbytes` counts 4 bytes per scale whatever dtype holds them, as the
    reference does (`webtorch/_core.py:4458-4459`)."""
    from webpytorch_amd import core, synth
    L = synth.gptq_layer(9, 256, 64, 128, 4)
    ql = core.QuantizedLinear.from_autogptq(L["qweight"], L["qzeros"], L["scales"], None, 128, 4)
    assert ql.scales.dtype.itemsize == 2
    assert ql.nbytes() == (32 * 64 + 2 * 8 + 2 * 64 + 64) * 4
