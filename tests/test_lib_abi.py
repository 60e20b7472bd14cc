"""The C ABI (CPU): libmiq.so loads, exports every function include/miq.h declares, the
Python binding covers them, and argument validation fails cleanly without touching a GPU."""
import ctypes
import os
import re

import pytest

from webpytorch_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "miq.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(miq_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "miq_gptq_gemv" in names and "miq_q4k_gemv" in names and len(names) >= 8


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing
    assert L.miq_version() == 1


def test_binding_covers_every_compute_entry_point():
    skip = {"miq_last_error", "miq_version", "miq_decode_state_words", "miq_gptq_gemv_noalloc_max_bytes"}
    assert set(declared_functions()) - skip == set(_lib.SIGNATURES)


def test_validation_errors_raise_without_gpu():
    # rejected before any HIP call: unsupported bit width, bad divisibility, bad Q4_K K
    with pytest.raises(NotImplementedError, match="bits=3"):
        _lib.call("miq_gptq_gemv", None, 1, None, None, None, None, 1, None, None, 1, 1, 64, 64, 32, 3, 0.0,
                  None, 0, None)
    with pytest.raises(ValueError, match="divide"):
        _lib.call("miq_gptq_gemv", None, 1, None, None, None, None, 1, None, None, 1, 1, 100, 64, 32, 4, 0.0,
                  None, 0, None)
    with pytest.raises(ValueError, match="multiple of 256"):
        _lib.call("miq_q4k_gemv", None, 1, None, None, None, 0, 1, 300, 8, None)
    with pytest.raises(ValueError, match="divide"):
        _lib.call("miq_gptq_quantize", None, 0, 0, 100, 8, 32, 4, None, None, None, None)
    msg = _lib.lib().miq_last_error().decode()
    assert "gptq_quantize" in msg


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libmiq.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.MiqError, match="not built"):
        _lib.lib()


def test_gemv_workspace_query_is_host_only():
    """The split-K plan is computed on the host: a K range longer than one workgroup's batches
    gets a workspace (counters + partials), a short one none."""
    from webpytorch_amd import core
    small = core.gemv_workspace_bytes(1, 896, 4864, 128, 4, _lib.MIQ_F16)
    assert small > 0 and small % 4 == 0
    assert small >= 4864 * 4 * 2  # at least two K slices of fp32 partials
    assert core.gemv_workspace_bytes(1, 128, 151936, 128, 4, _lib.MIQ_F16) == 0
    assert core.gemv_workspace_bytes(0, 896, 4864, 128, 4, _lib.MIQ_F16) == 0
    with pytest.raises(NotImplementedError, match="group size"):
        core.gemv_workspace_bytes(1, 896, 4864, 16, 4, _lib.MIQ_F16)
