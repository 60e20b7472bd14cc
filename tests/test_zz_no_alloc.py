"""GPU: `miq_gptq_gemv_noalloc` (the GEMV whose split-K workspace is the library's fixed device
array) gives the same bits as `miq_gptq_gemv` with a caller workspace, on two calls in a row
(the second smaller, reusing the array the first left behind), both matching the oracle; a
problem too large for the array fails before launching anything; a first call made under graph
capture is refused, and after one eager call captured calls replay correctly. Calls go through
the C ABI."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import gptq
from webpytorch_amd import synth

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _case(seed, M, K, N, xdt, bits=4, gs=128):
    import torch
    from webpytorch_amd import core
    L = synth.gptq_layer(seed, K, N, gs, bits)
    x = synth.activations(seed, M, K, xdt)
    dev = {k: core.to_device(L[k]) for k in ("qweight", "qzeros", "scales")}
    xt = core.to_device(x)
    bias = core.to_device(np.linspace(-1, 1, N).astype(np.float32))
    ref = gptq.gptq_matmul_np(x.astype(np.float32), L["qweight"], L["qzeros"], L["scales"], K, N, gs, bits, 1.0)
    ref = ref + np.linspace(-1, 1, N).astype(np.float32)
    return dev, xt, bias, ref, torch


def _call(name, dev, xt, bias, out, M, K, N, gs, bits, ws=None):
    from webpytorch_amd import _lib, core
    args = [_ptr(xt), core.dtype_code(xt), None, _ptr(dev["qweight"]), _ptr(dev["qzeros"]), _ptr(dev["scales"]),
            core.dtype_code(dev["scales"]), _ptr(bias), _ptr(out), core.dtype_code(out), M, K, N, gs, bits, 1.0]
    if name == "miq_gptq_gemv":
        args += [_ptr(ws) if ws is not None else None, 0 if ws is None else ws.numel()]
    args.append(core.stream_handle())
    _lib.call(name, *args)


@pytest.mark.parametrize("first,second", [((4, 4096, 4096, np.float16), (1, 896, 1152, np.float32)),
                                          ((1, 4096, 11008, np.float32), (1, 896, 4864, np.float16))])
def test_noalloc_matches_workspace_entry_point(gpu, first, second):
    from webpytorch_amd import core
    for seed, (M, K, N, xdt) in enumerate((first, second)):
        dev, xt, bias, ref, torch = _case(50 + seed, M, K, N, xdt)
        need = core.gemv_workspace_bytes(M, K, N, 128, 4, core.dtype_code(xt))
        assert 0 < need <= core._lib.lib().miq_gptq_gemv_noalloc_max_bytes()
        ws = torch.zeros(need, dtype=torch.uint8, device=xt.device)
        a = torch.empty((M, N), dtype=torch.float32, device=xt.device)
        b = torch.empty_like(a)
        print("case M=%d K=%d N=%d %s" % (M, K, N, np.dtype(xdt).name), flush=True)
        _call("miq_gptq_gemv", dev, xt, bias, a, M, K, N, 128, 4, ws)
        _call("miq_gptq_gemv_noalloc", dev, xt, bias, b, M, K, N, 128, 4)
        torch.cuda.synchronize()
        a, b = a.cpu().numpy(), b.cpu().numpy()
        assert np.array_equal(a, b)
        assert np.abs(b - ref).max() / np.abs(ref).max() < 1e-5
        assert np.all(np.abs(b - ref) <= 1e-3 + 1e-2 * np.abs(ref))


def test_noalloc_rejects_problems_beyond_the_array(gpu):
    import torch
    from webpytorch_amd import _lib, core
    M, K, N = 8, 16384, 65536
    assert core.gemv_workspace_bytes(M, K, N, 128, 4, _lib.MIQ_F32) > _lib.lib().miq_gptq_gemv_noalloc_max_bytes()
    x = torch.zeros((M, K), dtype=torch.float32, device="cuda")
    qw = torch.zeros((K // 8, N), dtype=torch.int32, device="cuda")
    qz = torch.zeros((K // 128, N // 8), dtype=torch.int32, device="cuda")
    sc = torch.zeros((K // 128, N), dtype=torch.float16, device="cuda")
    out = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="fixed scratch"):
        _lib.call("miq_gptq_gemv_noalloc", _ptr(x), 0, None, _ptr(qw), _ptr(qz), _ptr(sc), 1, None, _ptr(out), 0, M,
                  K, N, 128, 4, 1.0, core.stream_handle())
    torch.cuda.synchronize()
    assert not out.any()


_CAPTURE_CHILD = r"""
import ctypes, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from oracle import gptq
from webpytorch_amd import _lib, core, synth
L = _lib.lib()
M, K, N = 1, 896, 4864
lay = synth.gptq_layer(61, K, N, 128, 4)
x = synth.activations(61, M, K, np.float32)
dev = {k: core.to_device(lay[k]) for k in ("qweight", "qzeros", "scales")}
xt = core.to_device(x)
out = torch.zeros((M, N), dtype=torch.float32, device="cuda")
ref = gptq.gptq_matmul_np(x, lay["qweight"], lay["qzeros"], lay["scales"], K, N, 128, 4, 1.0)
s = torch.cuda.Stream()
P = lambda t: ctypes.c_void_p(t.data_ptr())
def call():
    return L.miq_gptq_gemv_noalloc(P(xt), 0, None, P(dev["qweight"]), P(dev["qzeros"]), P(dev["scales"]), 1, None,
                                   P(out), 0, M, K, N, 128, 4, 1.0, ctypes.c_void_p(s.cuda_stream))
def capture():
    g = ctypes.c_void_p()
    assert L.miq_graph_begin(ctypes.c_void_p(s.cuda_stream)) == 0
    rc = call()
    end = L.miq_graph_end(ctypes.c_void_p(s.cuda_stream), ctypes.byref(g))
    assert rc != 0 or end == 0
    return rc, g
torch.cuda.synchronize()
rc, g = capture()  # the process's first noalloc call, under capture: refused, nothing recorded
print("first captured call rc", rc, L.miq_last_error().decode(), flush=True)
assert rc == -1 and b"outside graph capture" in L.miq_last_error()
assert L.miq_graph_destroy(g) == 0
assert call() == 0  # one eager call sets the array up
s.synchronize()
rc, g = capture()
assert rc == 0
for rep in range(2):  # replays, with eager work on the device between them
    out.zero_()
    torch.cuda.synchronize()
    assert L.miq_graph_launch(g, ctypes.c_void_p(s.cuda_stream)) == 0
    s.synchronize()
    got = out.cpu().numpy()
    err = np.abs(got - ref).max() / np.abs(ref).max()
    print("replay", rep, "rel err", err, flush=True)
    assert err < 1e-5 and np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))
    torch.ones(1 << 20, device="cuda").sum().item()
assert L.miq_graph_destroy(g) == 0
print("ok", flush=True)
"""


def test_noalloc_first_call_under_capture_in_fresh_process(gpu):
    """In a fresh process: the first call under capture is refused (its one-time set-up cannot be
    recorded), an eager call then sets the array up, and a captured call replays twice matching
    the oracle."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root], capture_output=True, text=True, timeout=300)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and r.stdout.strip().endswith("ok")
