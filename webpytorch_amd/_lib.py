"""ctypes binding of libmiq.so (the C ABI declared in include/miq.h).

The library is loaded from this package directory only. There is no fallback: if it is
missing or does not load, every operator raises. Build it with
`python -m webpytorch_amd.build`.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmiq.so")

MIQ_F32, MIQ_F16 = 0, 1
MIQ_X_PLAIN, MIQ_X_RMSNORM, MIQ_X_SWIGLU = 0, 1, 2
ERRORS = {-1: ValueError, -2: ValueError, -3: NotImplementedError, -4: RuntimeError}

_p, _i, _f, _i64, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_int64, ctypes.c_size_t
_d = ctypes.c_double

# name -> argument types (restype is int for every compute entry point)
SIGNATURES = {
    "miq_graph_begin": [_p],
    "miq_graph_end": [_p, _p],
    "miq_graph_launch": [_p, _p],
    "miq_graph_destroy": [_p],
    "miq_gptq_dequant_f32": [_p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _f, _p],
    "miq_gptq_repack_rows": [_p, _p, _p, _i, _i, _i, _p],
    "miq_gptq_gemv_workspace": [_i, _i, _i, _i, _i, _i, _p],
    "miq_gptq_gemv": [_p, _i, _p, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _f, _p, _sz, _p],
    "miq_gptq_gemv_noalloc": [_p, _i, _p, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _f, _p],
    "miq_gptq_gemv_fused": [_p, _i, _p, _f, _p, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i, _f, _p, _sz, _p],
    "miq_gptq_gemm_workspace": [_i, _i, _i, _i, _i, _p],
    "miq_gptq_gemm": [_p, _p, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _f, _p, _sz, _p],
    "miq_gptq_gemm_f32x_workspace": [_i, _i, _i, _i, _i, _p],
    "miq_gptq_gemm_f32x": [_p, _p, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _f, _p, _sz, _p],
    "miq_gptq_quantize": [_p, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p],
    "miq_moe_route_bytes": [_i, _i, _i, _p],
    "miq_moe_route": [_p, _i, _i, _i, _i, _p, _sz, _p],
    "miq_moe_gate_up": [_p, _i, _p, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i, _p, _p, _p, _i, _i, _i, _i, _f, _p],
    "miq_moe_shared_add": [_p, _p, _p, _i, _i, _p],
    "miq_moe_down": [_p, _p, _i, _i, _i, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _f, _p],
    "miq_moe_combine": [_p, _p, _i, _i, _i, _p, _i, _p],
    "miq_moe_ggml_gemv": [_p, _i, _p, _i, _i, _i, _i, _i, _p, _i, _sz, _p, _i, _i, _p],
    "miq_q4k_gemm_workspace": [_i, _i, _i, _i, _p],
    "miq_q4k_gemm": [_p, _i, _p, _p, _p, _i, _i, _i, _i, _p, _sz, _p],
    "miq_ggml_gemm_workspace": [_i, _i, _i, _i, _i, _p],
    "miq_ggml_gemm": [_p, _i, _p, _i, _p, _p, _i, _i, _i, _i, _p, _sz, _p],
    "miq_embed": [_p, _p, _p, _i, _i, _i, _p],
    "miq_embed_f32": [_p, _p, _p, _i, _i, _i, _p],
    "miq_rmsnorm": [_p, _p, _p, _i, _i, _f, _p],
    "miq_head_rmsnorm": [_p, _p, _p, _i, _i, _i, _i, _f, _p],
    "miq_rope_kv": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p],
    "miq_attention_decode": [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _f, _p],
    "miq_attention": [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _f, _p],
    "miq_silu_mul": [_p, _p, _i, _i, _p],
    "miq_add": [_p, _p, _i64, _p],
    "miq_argmax_advance": [_p, _i, _p, _p, _i, _p, _i, _p],
    "miq_q4k_dequant_f32": [_p, _p, _i64, _p],
    "miq_decode_persistent_plan": [_i] * 10 + [_p, _p],
    "miq_decode_persistent": [_p] * 10 + [_i, _p, _p, _p, _sz] + [_i] * 10 + [_f] * 3 + [_p],
    "miq_decode_persistent_trace": [_p] * 10 + [_i, _p, _p, _p, _sz] + [_i] * 10 + [_f] * 3 + [_p, _sz, _p],
    "miq_q4k_gemv": [_p, _i, _p, _p, _p, _i, _i, _i, _i, _p],
    "miq_ggml_gemv": [_p, _i, _p, _i, _p, _p, _i, _i, _i, _i, _p],
    "miq_ggml_dequant_f32": [_p, _i, _p, _i64, _p],
}

_lib = None


class MiqError(RuntimeError):
    pass


def lib():
    """Load libmiq.so once; raise if it is absent (no CPU fallback exists)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MiqError("libmiq.so is not built (%s); run `python -m webpytorch_amd.build`"
                           % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        L.miq_last_error.restype = ctypes.c_char_p
        L.miq_last_error.argtypes = []
        L.miq_version.restype = ctypes.c_int
        L.miq_decode_state_words.restype = ctypes.c_int
        L.miq_decode_state_words.argtypes = []
        L.miq_gptq_gemv_noalloc_max_bytes.restype = ctypes.c_size_t
        L.miq_gptq_gemv_noalloc_max_bytes.argtypes = []
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        _lib = L
    return _lib


def call(name, *args):
    """Invoke an entry point and turn a negative return code into a Python exception."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().miq_last_error().decode(errors="replace")
        raise ERRORS.get(rc, MiqError)("%s failed (%d): %s" % (name, rc, msg))
    return rc
