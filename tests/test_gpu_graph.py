"""GPU: capture and replay through the C ABI (`miq_graph_begin/end/launch/destroy`, the
reference's beginCapture / endCapture / replay, `webtorch/platform.py:45-56`). A one-token
head step (int4 GEMV to the logits, then the greedy pick that advances the device state) is
recorded on a side stream and replayed several times, with eager work and synchronisations
between the replays; every replay must equal the eager launches bit for bit."""
import ctypes

import numpy as np
import pytest

from webpytorch_amd import synth

pytestmark = pytest.mark.gpu


def _head_step(core, _lib, x, L, logits, ids, hist, state, ws, K, N, stream):
    _lib.call("miq_gptq_gemv", core.ptr(x), core.dtype_code(x), None, core.ptr(L["qw"]), core.ptr(L["qz"]),
              core.ptr(L["sc"]), core.dtype_code(L["sc"]), None, core.ptr(logits), core.dtype_code(logits),
              1, K, N, 128, 4, 0.0, core.ptr(ws), ws.numel(), stream)
    _lib.call("miq_argmax_advance", core.ptr(logits), N, core.ptr(ids), core.ptr(hist), hist.numel(),
              core.ptr(state), 1, stream)


def test_capture_replay_matches_eager(gpu):
    import torch
    from webpytorch_amd import _lib, core
    K, N = 896, 4864
    W = synth.gptq_layer(11, K, N, 128, 4)
    L = {"qw": torch.from_numpy(W["qweight"]).cuda(), "qz": torch.from_numpy(W["qzeros"]).cuda(),
         "sc": torch.from_numpy(W["scales"]).cuda()}
    xs = [torch.from_numpy(synth.activations(20 + i, 1, K, np.float32)).cuda() for i in range(4)]
    ws = core.workspace(core.gemv_workspace_bytes(1, K, N, 128, 4, core.dtype_code(xs[0])))

    def buffers():
        return (torch.empty((1, N), dtype=torch.float32, device="cuda"),
                torch.zeros(1, dtype=torch.int32, device="cuda"),
                torch.full((8,), -1, dtype=torch.int32, device="cuda"),
                torch.zeros(_lib.lib().miq_decode_state_words(), dtype=torch.int32, device="cuda"))

    # eager: one step per input, state carried across the steps
    e_logits, e_ids, e_hist, e_state = buffers()
    want = []
    for x in xs:
        _head_step(core, _lib, x, L, e_logits, e_ids, e_hist, e_state, ws, K, N, core.stream_handle())
        torch.cuda.synchronize()
        want.append((e_logits.clone(), e_ids.clone(), e_state.clone()))
    assert torch.equal(e_hist[:4].cpu(), torch.stack([w[1][0] for w in want]).cpu())

    # recorded once on a side stream; the input buffer is refilled eagerly before each replay
    x = torch.empty_like(xs[0])
    logits, ids, hist, state = buffers()
    side = torch.cuda.Stream()
    sh = ctypes.c_void_p(side.cuda_stream)
    torch.cuda.synchronize()
    graph = ctypes.c_void_p()
    _lib.call("miq_graph_begin", sh)
    try:
        _head_step(core, _lib, x, L, logits, ids, hist, state, ws, K, N, sh)
    finally:
        _lib.call("miq_graph_end", sh, ctypes.byref(graph))
    try:
        assert graph.value
        torch.cuda.synchronize()
        assert not state.any()  # nothing ran while recording
        for i, x_i in enumerate(xs):
            x.copy_(x_i)
            logits.fill_(float("nan"))
            torch.cuda.synchronize()
            _lib.call("miq_graph_launch", graph, sh)
            side.synchronize()
            wl, wi, wst = want[i]
            assert torch.equal(logits, wl), f"replay {i}: logits differ from the eager launch"
            assert torch.equal(ids, wi) and torch.equal(state, wst), f"replay {i}: state differs"
        assert torch.equal(hist, e_hist)
    finally:
        _lib.call("miq_graph_destroy", graph)


def test_graph_errors_are_reported(gpu):
    import torch
    from webpytorch_amd import _lib, core
    with pytest.raises(ValueError, match="null stream"):
        _lib.call("miq_graph_begin", None)
    with pytest.raises(ValueError, match="null graph"):
        _lib.call("miq_graph_launch", None, None)
    _lib.call("miq_graph_destroy", None)
    # ending a recording that was never begun fails with the runtime's reason, and leaves no
    # error behind for the next launch
    side = torch.cuda.Stream()
    graph = ctypes.c_void_p()
    with pytest.raises(RuntimeError, match="graph_end"):
        _lib.call("miq_graph_end", ctypes.c_void_p(side.cuda_stream), ctypes.byref(graph))
    assert not graph.value
    x = torch.ones((1, 8), device="cuda")
    out = torch.empty((1, 8), device="cuda")
    _lib.call("miq_add", core.ptr(out.copy_(x)), core.ptr(x), 8, core.stream_handle())
    torch.cuda.synchronize()
    assert torch.equal(out, 2 * x)
