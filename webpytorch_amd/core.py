"""Quantized linear operators on MI355X: drop-in counterparts of the reference's
`QuantizedLinear`, `GGMLLinear`, `_gptq_matmul`, `ggml_matmul`, `ggml_native_supported` and
`_gptq_quantize` (`webtorch/_core.py:3644-3824, 4008-4043, 4377-4459`).

Host code is PyTorch-ROCm: torch owns device memory and the current HIP stream, and every
operator enqueues hand-written HIP kernels from libmiq.so through its C ABI. There is no CPU
path: without the library (or without a GPU) every call raises.

Tensors may be given as numpy arrays (uploaded once, at construction) or torch tensors. The
weight layouts are the reference's: qweight int32 (K/per, N), qzeros int32 (K/gs, N/per),
scales (K/gs, N), Q4_K rows of 144-byte super-blocks.
"""
import ctypes

import numpy as np
import torch

from . import _lib
from ._lib import MIQ_F16, MIQ_F32

# M above which a GPTQ matmul leaves the GEMV kernel for the MFMA GEMM.
GEMV_MAX_M = 8


# ---- plumbing --------------------------------------------------------------------------
def device():
    if not torch.cuda.is_available():
        raise RuntimeError("webpytorch_amd needs a ROCm GPU (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def stream_handle():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def dtype_code(t):
    if t.dtype == torch.float16:
        return MIQ_F16
    if t.dtype == torch.float32:
        return MIQ_F32
    raise TypeError("unsupported dtype %s (float16 or float32)" % t.dtype)


def to_device(a, dtype=None):
    """numpy / torch -> contiguous tensor on the current GPU (no copy if already there)."""
    if isinstance(a, torch.Tensor):
        t = a
    else:
        arr = np.ascontiguousarray(a)
        if arr.dtype == np.uint32:
            arr = arr.view(np.int32)
        t = torch.from_numpy(arr)
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.to(device()).contiguous()


def as_activation(x):
    """Activation tensor on the GPU as float16 or float32 (other dtypes become float32)."""
    t = getattr(x, "data", x) if not isinstance(x, (torch.Tensor, np.ndarray)) else x
    t = to_device(t)
    if t.dtype not in (torch.float16, torch.float32):
        t = t.float()
    return t


_WORKSPACE = {}
_RETIRED = {}
_WS_BYTES = {}


def gemv_workspace_bytes(M, K, N, gs, bits, x_dtype):
    """Bytes of split-K workspace the GEMV needs for this problem (cached per shape)."""
    key = (M, K, N, gs, bits, x_dtype)
    b = _WS_BYTES.get(key)
    if b is None:
        n = ctypes.c_size_t(0)
        _lib.call("miq_gptq_gemv_workspace", M, K, N, gs, bits, x_dtype, ctypes.byref(n))
        b = _WS_BYTES[key] = int(n.value)
    return b


def gemm_f32x_workspace_bytes(M, K, N, gs, bits):
    """Bytes of workspace the fp32-activation GEMM needs (cached per shape)."""
    key = ("gemm32", M, K, N, gs, bits)
    b = _WS_BYTES.get(key)
    if b is None:
        n = ctypes.c_size_t(0)
        _lib.call("miq_gptq_gemm_f32x_workspace", M, K, N, gs, bits, ctypes.byref(n))
        b = _WS_BYTES[key] = int(n.value)
    return b


def gemm_workspace_bytes(M, K, N, gs, bits):
    """Bytes of split-K workspace the MFMA GEMM needs for this problem (cached per shape)."""
    key = ("gemm", M, K, N, gs, bits)
    b = _WS_BYTES.get(key)
    if b is None:
        n = ctypes.c_size_t(0)
        _lib.call("miq_gptq_gemm_workspace", M, K, N, gs, bits, ctypes.byref(n))
        b = _WS_BYTES[key] = int(n.value)
    return b


def workspace(nbytes):
    """The split-K workspace of the current (device, stream), grown on demand and zeroed when
    allocated (the kernels leave its counter region zero). One workspace per stream: calls on
    one stream are ordered, so they never share it concurrently, and calls on two streams get
    two workspaces. A grown workspace keeps the old one alive (a captured graph may still point
    at it); growth at least doubles, so a stream retires O(log size) buffers."""
    if nbytes == 0:
        return None
    dev = torch.cuda.current_device()
    key = (dev, torch.cuda.current_stream(dev).cuda_stream)
    t = _WORKSPACE.get(key)
    if t is None or t.numel() < nbytes:
        size = max(nbytes, 8 << 20)
        if t is not None:
            _RETIRED.setdefault(key, []).append(t)
            size = max(size, 2 * t.numel())
        t = torch.zeros(size, dtype=torch.uint8, device=device())
        _WORKSPACE[key] = t
    return t


def aligned16(t):
    """The kernels read activations with 16-byte loads: copy a misaligned view."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _scales(s):
    t = to_device(s)
    return t if t.dtype in (torch.float16, torch.float32) else t.float()


# ---- first-use known-answer checks ---------------------------------------------------
# The reference multiplies one random block per (ggml type, kernel mode) the first time that
# kernel runs and raises if it disagrees with the dequantizer (`_ggml_selfcheck`,
# `webtorch/_core.py:3684-3717`), so that a broken build raises instead of producing plausible
# numbers. The same is done here for every product path, on the device: the kernel's result for
# a small random problem against the exact fp32 dequant (its own kernel, bit-exact) times x,
# accumulated in float64. Each (path, device) is checked once, outside graph capture.
_CHECKED = set()
SELFCHECK_RTOL = 1e-4


def _first_use(key):
    """True (and the key recorded) if `key` has not been checked on this device yet and the
    current stream is not capturing a graph (a check reads its result back to the host)."""
    k = key + (torch.cuda.current_device(),)
    if k in _CHECKED or torch.cuda.is_current_stream_capturing():
        return False
    _CHECKED.add(k)
    return True


def _reference_product(x, W):
    """x (M, K) @ W (K, N) in float64 on the device."""
    return x.double() @ W.double()


def _check_close(what, got, want):
    err = float((got.double() - want).abs().max() / (want.abs().max() + 1e-30))
    if not err < SELFCHECK_RTOL:
        raise RuntimeError("%s is wrong on this device (rel err %.3g against the exact dequant)" % (what, err))


def _selfcheck_gptq(M, xdt, bits, gs, sdt=torch.float16, zoff=1.0):
    """Known-answer check of the kernel `_gptq_matmul` picks for M rows of `xdt` activations,
    with scales of dtype `sdt` and zero offset `zoff` (each pair is its own instantiation)."""
    g = np.random.default_rng(0x5e1f + M + 31 * bits)
    K, N = 256, 256
    per = 32 // bits
    qw = torch.from_numpy(g.integers(0, 1 << 32, (K // per, N), dtype=np.uint64).astype(np.uint32).view(np.int32))
    qz = torch.from_numpy(g.integers(0, 1 << 32, (K // gs, N // per), dtype=np.uint64).astype(np.uint32).view(np.int32))
    sc = torch.from_numpy((np.abs(g.standard_normal((K // gs, N))) * 0.01 + 1e-3).astype(np.float32)).to(sdt)
    x = torch.from_numpy(g.standard_normal((M, K)).astype(np.float32)).to(device(), xdt)
    qw, qz, sc = qw.to(device()), qz.to(device()), sc.to(device())
    got = _gptq_matmul(x, qw, qz, sc, K, N, gs, bits, zoff, out_dtype=torch.float32, _check=False)
    want = _reference_product(x, gptq_dequant(qw, qz, sc, K, N, gs, bits, zoff))
    _check_close("the GPTQ int%d product kernel for %d rows of %s (%s scales, zero offset %g)" % (
        bits, M, str(xdt).replace("torch.", ""), str(sdt).replace("torch.", ""), zoff), got, want)


def selfcheck_gptq(M, xdt, bits, gs, sdt, zoff):
    """Run the first-use check of the product class for (M rows of xdt, bits, gs, scales dtype,
    zero offset) now, if it has not run on this device: for callers about to capture a graph,
    where checks are skipped."""
    if M and 256 % gs == 0 and _first_use(("gptq", bits, gs, _gptq_path(M, xdt), xdt, sdt, float(zoff))):
        _selfcheck_gptq(_gptq_path(M, xdt), xdt, bits, gs, sdt, float(zoff))


def _gptq_path(M, xdt):
    """The product kernel class `_gptq_matmul` runs for M rows (one check per class)."""
    if M == 1:
        return 1
    if M <= GEMV_MAX_M:
        return 4
    return 12 if M <= 16 and xdt == torch.float16 else 40


# ---- GPTQ ----------------------------------------------------------------------------
def gptq_dequant(qweight, qzeros, scales, K, N, gs, bits, zoff=0.0, g_idx=None):
    """Full fp32 weight (K, N); bit-exact with the reference's dequant for integer zoff."""
    out = torch.empty((K, N), dtype=torch.float32, device=device())
    _lib.call("miq_gptq_dequant_f32", ptr(qweight), ptr(qzeros), ptr(scales), dtype_code(scales),
              ptr(g_idx), ptr(out), K, N, gs, bits, float(zoff), stream_handle())
    return out


def _gptq_matmul(xf, qweight, qzeros, scales, K, N, gs, bits, zoff=0.0, *, bias=None, perm=None,
                 out_dtype=None, out=None, ws=None, _check=True):
    """xf (M, K) @ dequant(W) (+ bias) -> (M, N) on the current stream
    (`webtorch/_core.py:4008-4043`). Up to GEMV_MAX_M rows run the split-K GEMV; more rows
    run the matrix-core GEMM (fp32 activations as row-scaled fp16 hi/lo pairs of rows). The
    first call of each kernel class on a device runs its known-answer check (RuntimeError if
    it fails)."""
    M = int(xf.shape[0])
    if _check:
        selfcheck_gptq(M, xf.dtype, bits, gs, scales.dtype, zoff)
    od = out_dtype or torch.float32
    if out is None:
        out = torch.empty((M, N), dtype=od, device=xf.device)
    if M == 0:
        return out
    xf = aligned16(xf)
    xd = dtype_code(xf)
    if M > GEMV_MAX_M and xd == MIQ_F16 and float(zoff).is_integer() and 0 <= zoff <= 8:
        if ws is None:
            ws = workspace(gemm_workspace_bytes(M, K, N, gs, bits))
        _lib.call("miq_gptq_gemm", ptr(xf), ptr(perm), ptr(qweight), ptr(qzeros), ptr(scales),
                  dtype_code(scales), ptr(bias), ptr(out), dtype_code(out), M, K, N, gs, bits,
                  float(zoff), ptr(ws), 0 if ws is None else ws.numel(), stream_handle())
        return out
    if M > GEMV_MAX_M and float(zoff).is_integer() and 0 <= zoff <= 8 and K <= 32768:
        need = gemm_f32x_workspace_bytes(M, K, N, gs, bits)
        if ws is None or ws.numel() < need:
            ws = workspace(need)
        _lib.call("miq_gptq_gemm_f32x", ptr(xf), ptr(perm), ptr(qweight), ptr(qzeros), ptr(scales),
                  dtype_code(scales), ptr(bias), ptr(out), dtype_code(out), M, K, N, gs, bits,
                  float(zoff), ptr(ws), ws.numel(), stream_handle())
        return out
    if ws is None:
        ws = workspace(gemv_workspace_bytes(M, K, N, gs, bits, xd))
    _lib.call("miq_gptq_gemv", ptr(xf), xd, ptr(perm), ptr(qweight), ptr(qzeros),
              ptr(scales), dtype_code(scales), ptr(bias), ptr(out), dtype_code(out), M, K, N, gs,
              bits, float(zoff), ptr(ws), 0 if ws is None else ws.numel(), stream_handle())
    return out


def gptq_quantize(W, group_size=32, bits=4, from_out_in=False):
    """Device quantizer, bit-exact with `_gptq_quantize` (`webtorch/_core.py:3782-3824`).
    W (K, N) or (N, K) with from_out_in, float16/float32. Returns (qweight, qzeros, scales
    float32, K, N) as GPU tensors."""
    Wt = as_activation(W)
    K, N = (Wt.shape[1], Wt.shape[0]) if from_out_in else Wt.shape
    per = 32 // bits
    if K % group_size or K % per or N % per:
        raise AssertionError("dims must divide group/pack size")
    qw = torch.empty((K // per, N), dtype=torch.int32, device=Wt.device)
    qz = torch.empty((K // group_size, N // per), dtype=torch.int32, device=Wt.device)
    sc = torch.empty((K // group_size, N), dtype=torch.float32, device=Wt.device)
    _lib.call("miq_gptq_quantize", ptr(Wt), dtype_code(Wt), int(bool(from_out_in)), K, N, group_size,
              bits, ptr(qw), ptr(qz), ptr(sc), stream_handle())
    return qw, qz, sc, K, N


def act_order_perm(g_idx, gs):
    """Stable argsort of g_idx (host, load time): groups become consecutive runs of gs rows.
    Raises if g_idx does not hold exactly gs rows per group."""
    g = np.asarray(g_idx.cpu() if isinstance(g_idx, torch.Tensor) else g_idx).astype(np.int64)
    perm = np.argsort(g, kind="stable")
    if np.any(g[perm] != np.arange(g.size) // gs):
        raise ValueError("g_idx must assign exactly group_size rows to every group")
    return perm.astype(np.int32)


class QuantizedLinear:
    """Inference-only GPTQ-format weight-quantized Linear (group-wise int4/int8), same
    constructor and attributes as the reference (`webtorch/_core.py:4409-4459`).

    Differences, all invisible to results: scales stay in the dtype they are given (fp16
    AutoGPTQ scales are not widened to fp32; both dequantize to identical values), the bias
    is fused into the kernel, and an optional `g_idx` (act-order, which the reference ignores)
    is honoured by a load-time row repack plus an activation gather."""

    def __init__(self, qweight, qzeros, scales, bias, Kt, Nt, Kp, Np, gs, bits, zero_offset=0.0,
                 g_idx=None):
        self.Kt, self.Nt, self.Kp, self.Np = int(Kt), int(Nt), int(Kp), int(Np)
        self.gs, self.bits = int(gs), int(bits)
        self.zero_offset = float(zero_offset)
        per = 32 // self.bits
        if self.Kp % self.gs or self.Kp % per or self.Np % per:
            raise AssertionError("dims must divide group/pack size")
        self.qweight = to_device(qweight, torch.int32)
        self.qzeros = to_device(qzeros, torch.int32)
        self.scales = _scales(scales)
        if tuple(self.qweight.shape) != (self.Kp // per, self.Np):
            raise ValueError("qweight shape %s != (%d, %d)" % (tuple(self.qweight.shape), self.Kp // per, self.Np))
        b = torch.zeros(self.Np, dtype=torch.float32)
        if bias is not None:
            bb = torch.as_tensor(np.asarray(bias.cpu() if isinstance(bias, torch.Tensor) else bias, np.float32))
            b[:bb.numel()] = bb.reshape(-1)
        self.bias = b.to(device())
        self.perm = None
        self.g_idx = None
        if g_idx is not None:
            gi = np.asarray(g_idx.cpu() if isinstance(g_idx, torch.Tensor) else g_idx).astype(np.int64)
            if np.any(gi != np.arange(gi.size) // self.gs):
                perm = act_order_perm(gi, self.gs)
                self.g_idx = to_device(gi.astype(np.int32))
                self.perm = to_device(perm)
                rep = torch.empty_like(self.qweight)
                _lib.call("miq_gptq_repack_rows", ptr(self.qweight), ptr(self.perm), ptr(rep),
                          self.Kp, self.Np, self.bits, stream_handle())
                self.qweight = rep

    @staticmethod
    def from_autogptq(qweight, qzeros, scales, bias, gs, bits, g_idx=None):
        """AutoGPTQ tensors (`webtorch/_core.py:4420-4430`): zero points use the +1
        convention (zero_offset 1.0). `g_idx` (desc_act=True) is an extension."""
        per = 32 // bits
        K = int(np.shape(qweight)[0]) * per
        N = int(np.shape(qweight)[1])
        return QuantizedLinear(qweight, qzeros, scales, bias, K, N, K, N, gs, bits, zero_offset=1.0,
                               g_idx=g_idx)

    @staticmethod
    def from_linear(lin, group_size=32, bits=4):
        """Quantize a float Linear whose weight is (in, out) = (K, N), as the reference's
        `Linear` stores it (`webtorch/_core.py:4433-4444`), on the device."""
        W = to_device(getattr(lin.weight, "data", lin.weight)).float()
        bsrc = getattr(lin, "bias", None)
        b = None if bsrc is None else to_device(getattr(bsrc, "data", bsrc)).float()
        K, N = W.shape
        per = 32 // bits
        kmul = group_size if group_size % per == 0 else group_size * per
        Kp, Np = K + (-K) % kmul, N + (-N) % per
        if Kp != K or Np != N:
            W = torch.nn.functional.pad(W, (0, Np - N, 0, Kp - K))
        qw, qz, sc, _, _ = gptq_quantize(W, group_size, bits)
        return QuantizedLinear(qw, qz, sc, b, K, N, Kp, Np, group_size, bits)

    def forward(self, x, out_dtype=torch.float32):
        """x (..., Kt) -> (..., Nt), float32 like the reference's `forward` (its
        `_gptq_matmul` accumulates and returns fp32); `out_dtype=torch.float16` writes fp16
        from the kernel instead."""
        xt = as_activation(x)
        lead = xt.shape[:-1]
        xf = xt.reshape(-1, self.Kt)
        if self.Kp != self.Kt:
            xf = torch.nn.functional.pad(xf, (0, self.Kp - self.Kt))
        xf = xf.contiguous()
        of = _gptq_matmul(xf, self.qweight, self.qzeros, self.scales, self.Kp, self.Np, self.gs,
                          self.bits, self.zero_offset, bias=self.bias, perm=self.perm,
                          out_dtype=out_dtype)
        if self.Np != self.Nt:
            of = of[:, :self.Nt].contiguous()
        return of.reshape(*lead, self.Nt)

    __call__ = forward

    def dequantize(self):
        """fp32 (Kp, Np) weight in the original row order."""
        if self.perm is None:
            return gptq_dequant(self.qweight, self.qzeros, self.scales, self.Kp, self.Np, self.gs,
                                self.bits, self.zero_offset)
        W = gptq_dequant(self.qweight, self.qzeros, self.scales, self.Kp, self.Np, self.gs, self.bits,
                         self.zero_offset)
        out = torch.empty_like(W)
        out[self.perm.long()] = W
        return out

    def nbytes(self):
        """The reference's count (`webtorch/_core.py:4458-4459`): int32 qweight and qzeros, fp32
        scales and bias -- 4 bytes each, whatever dtype the scales are held in here."""
        return int(self.qweight.numel() * 4 + self.qzeros.numel() * 4 + self.scales.numel() * 4 +
                   self.bias.numel() * 4)


# ---- GGUF native ---------------------------------------------------------------------
# (values per block, bytes per block, ggml type id) of the types a native kernel decodes
_NATIVE_TYPES = {"Q4_K": (256, 144, 12), "Q6_K": (256, 210, 14), "Q8_0": (32, 34, 8),
                 "Q4_0": (32, 18, 2), "Q4_1": (32, 20, 3), "Q5_0": (32, 22, 6), "Q5_1": (32, 24, 7),
                 "IQ4_NL": (32, 18, 20), "IQ4_XS": (256, 136, 23), "Q5_K": (256, 176, 13),
                 "Q2_K": (256, 84, 10), "Q3_K": (256, 110, 11),
                 "IQ2_XXS": (256, 66, 16), "IQ2_XS": (256, 74, 17), "IQ2_S": (256, 82, 22),
                 "IQ3_XXS": (256, 98, 18), "IQ3_S": (256, 110, 21), "IQ1_S": (256, 50, 19),
                 "IQ1_M": (256, 56, 29), "TQ1_0": (256, 54, 34), "TQ2_0": (256, 66, 35),
                 "MXFP4": (32, 17, 39), "NVFP4": (64, 36, 40), "Q1_0": (128, 18, 41), "Q2_0": (64, 18, 42),
                 "F32": (1, 4, 0), "F16": (1, 2, 1), "BF16": (1, 2, 30)}
# types a 2-D weight is stored in without quantization (multiplied as stored)
DENSE_TYPES = ("F32", "F16", "BF16")


def ggml_native_supported(type_name):
    """Can this ggml type be multiplied straight from the file's bytes
    (`webtorch/_core.py:3644-3646`, table 3609-3637)? Every type of the reference's table is:
    the K-quants and legacy block types, the codebook-grid i-quants (IQ1_S, IQ1_M, IQ2_XXS,
    IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ4_NL, IQ4_XS), the ternary TQ1_0 / TQ2_0, the fp4 MXFP4 /
    NVFP4, Q1_0 / Q2_0, and unquantized F32 / F16 / BF16 matrices."""
    return type_name in _NATIVE_TYPES


def q4k_dequant(blocks, n_blocks):
    out = torch.empty(int(n_blocks) * 256, dtype=torch.float32, device=blocks.device)
    _lib.call("miq_q4k_dequant_f32", ptr(blocks), ptr(out), int(n_blocks), stream_handle())
    return out


def ggml_dequant(blocks, type_name, n_blocks):
    """fp32 values of n_blocks blocks of a native type, bit-exact with `ggufload.dequant`
    (`webtorch/ggufload.py:133-222`)."""
    if type_name not in _NATIVE_TYPES:
        raise NotImplementedError("native ggml type %s" % type_name)
    vals, _, tid = _NATIVE_TYPES[type_name]
    out = torch.empty(int(n_blocks) * vals, dtype=torch.float32, device=blocks.device)
    _lib.call("miq_ggml_dequant_f32", ptr(blocks), tid, ptr(out), int(n_blocks), stream_handle())
    return out


def _row_bytes(type_name, K):
    vals, blk, _ = _NATIVE_TYPES[type_name]
    if K % vals:
        raise ValueError("K=%d is not a multiple of the %s block (%d values)" % (K, type_name, vals))
    return K // vals * blk


def ggml_transpose(src, n, rowb):
    """Load-time layout step, same name and arguments as the reference's (`(n, rowb bytes)` in,
    `webtorch/_core.py:4315-4344`), returning the layout the kernels here read: the n rows of
    rowb bytes unchanged, as a uint8 (n, rowb) device tensor. The reference transposes to
    (word, row) u32 so that WebGPU threads read adjacent words; on MI355X a wave's 16-byte loads
    of the native rows already coalesce, so the bytes stay as the file holds them."""
    t = src if isinstance(src, torch.Tensor) else torch.from_numpy(
        np.frombuffer(bytearray(src), np.uint8) if isinstance(src, (bytes, bytearray))
        else np.ascontiguousarray(src).reshape(-1).view(np.uint8))
    b = t.reshape(-1).view(torch.uint8)
    if b.numel() < n * rowb:
        raise ValueError("%d bytes given, (%d, %d) needs %d" % (b.numel(), n, rowb, n * rowb))
    return b[:n * rowb].to(device()).contiguous().reshape(n, rowb)


def rows_from_transposed(words, n, rowb):
    """The reference's (word, row) u32 layout (`ggml_transpose` output: word w of row r at
    index w * n + r) back to n rows of rowb bytes, on the device."""
    nw = (rowb + 3) // 4
    w = words.reshape(-1)
    if w.numel() != nw * n:
        raise ValueError("transposed layout holds %d words, (%d rows x %d words) expected" % (w.numel(), n, nw))
    rows = w.view(torch.int32).reshape(nw, n).t().contiguous().view(torch.uint8).reshape(n, nw * 4)
    return rows[:, :rowb].contiguous()


# Q4_K rows above this count go to the matrix-core GEMM (the other types stay on the GEMV)
GGML_GEMV_MAX_M = 8


# Types whose rows above GGML_GEMV_MAX_M run on the matrix cores (`miq_ggml_gemm`), for K a
# multiple of 256: the four types of a Q4_K_M / Q5_K_M file
GGML_GEMM_TYPES = ("Q4_K", "Q5_K", "Q6_K", "Q8_0")


def ggml_gemm_workspace_bytes(M, K, N, x_dtype, type_name="Q4_K"):
    key = ("ggmlgemm", M, K, N, x_dtype, type_name)
    b = _WS_BYTES.get(key)
    if b is None:
        n = ctypes.c_size_t(0)
        _lib.call("miq_ggml_gemm_workspace", M, K, N, x_dtype, _NATIVE_TYPES[type_name][2], ctypes.byref(n))
        b = _WS_BYTES[key] = int(n.value)
    return b


def q4k_gemm_workspace_bytes(M, K, N, x_dtype):
    return ggml_gemm_workspace_bytes(M, K, N, x_dtype, "Q4_K")


def _ggml_gemm_taken(type_name, M, K):
    return type_name in GGML_GEMM_TYPES and M > GGML_GEMV_MAX_M and K % 256 == 0


def _ggml_selfcheck(type_name, mode):
    """Multiply two random blocks of `type_name` with the kernel of `mode` (rows 1, 2, 0 for 3
    to GGML_GEMV_MAX_M, -1 for the matrix-core GEMM) and compare against the device's exact dequant of the same bytes times x in
    float64; RuntimeError on a mismatch (`_ggml_selfcheck`, `webtorch/_core.py:3684-3717`).
    Code and sub-scale bytes are uniform random (every byte pattern is a legal block); the fp16
    scale fields are drawn small and finite, where the reference redraws until they are."""
    from . import synth
    vals = _NATIVE_TYPES[type_name][0]
    K = vals if vals > 1 else 72  # an unquantized row: 72 values (a ragged count of 16-byte words)
    if mode < 0:
        K = 256  # the GEMM walks K in 256-value steps (8 blocks of a 32-value type)
    raw = torch.from_numpy(synth.ggml_layer(type_name, 0, K, 2, scale=0.01)).to(device())
    W = ggml_dequant(raw.reshape(-1), type_name, 2 * K // vals).reshape(2, K)
    g = np.random.default_rng(vals)
    M = {0: 3, -1: 2 * GGML_GEMV_MAX_M + 1}.get(mode, mode)
    x = torch.from_numpy(g.standard_normal((M, K)).astype(np.float32)).to(device())
    got = ggml_matmul(x, raw, type_name, K, 2, _check=False)
    _check_close("the native ggml %s kernel for %s" % ("gemm" if mode < 0 else "gemv", type_name), got,
                 _reference_product(x, W.t()))


def ggml_matmul(xf, packed, type_name, K, N, bias=None, out_dtype=torch.float32, out=None, _check=True):
    """xf (M, K) @ W.T -> (M, N), decoding ggml blocks in the kernel
    (`webtorch/_core.py:3720-3734`).

    `packed` is either the layout `ggml_transpose` here returns (uint8 bytes: N rows of
    K / block-values blocks, as the file stores them) or the reference's own transposed
    (word, row) layout as int32/uint32 words, which is converted to rows on the device on every
    call (a copy of the weight: build a `GGMLLinear`, or pass rows, to avoid it). The dtype
    tells the two apart: bytes are rows, 32-bit words are the reference's transposed layout."""
    if type_name not in _NATIVE_TYPES:
        raise NotImplementedError("native ggml type %s" % type_name)
    rowb = _row_bytes(type_name, int(K))
    if not isinstance(packed, torch.Tensor):
        packed = to_device(packed)
    if packed.dtype in (torch.int32, torch.uint32):
        packed = rows_from_transposed(packed.to(device()), int(N), rowb)
    elif packed.dtype != torch.uint8:
        raise TypeError("packed must be uint8 rows or int32 transposed words, got %s" % packed.dtype)
    elif packed.numel() != int(N) * rowb:
        raise ValueError("packed holds %d bytes, %s (%d x %d) needs %d" % (packed.numel(), type_name, N, K,
                                                                           int(N) * rowb))
    xf = aligned16(as_activation(xf).contiguous())
    M = int(xf.shape[0])
    gemm = _ggml_gemm_taken(type_name, M, int(K))
    mode = -1 if gemm else (M if M <= 2 else 0)
    if _check and M and _first_use(("ggml", type_name, mode)):
        _ggml_selfcheck(type_name, mode)
    if out is None:
        out = torch.empty((M, N), dtype=out_dtype, device=xf.device)
    if gemm:  # prefill rows on the matrix cores
        need = ggml_gemm_workspace_bytes(M, int(K), int(N), dtype_code(xf), type_name)
        ws = workspace(need)
        _lib.call("miq_ggml_gemm", ptr(xf), dtype_code(xf), ptr(packed), _NATIVE_TYPES[type_name][2], ptr(bias),
                  ptr(out), dtype_code(out), M, int(K), int(N), ptr(ws), ws.numel(), stream_handle())
    elif type_name == "Q4_K":
        _lib.call("miq_q4k_gemv", ptr(xf), dtype_code(xf), ptr(packed), ptr(bias), ptr(out), dtype_code(out),
                  M, int(K), int(N), stream_handle())
    else:
        _lib.call("miq_ggml_gemv", ptr(xf), dtype_code(xf), ptr(packed), _NATIVE_TYPES[type_name][2], ptr(bias),
                  ptr(out), dtype_code(out), M, int(K), int(N), stream_handle())
    return out


class GGMLLinear:
    """Inference-only Linear whose weight stays in the GGUF encoding
    (`webtorch/_core.py:4377-4406`). The reference transposes the bytes to a (word, row)
    layout at upload for WebGPU coalescing; on MI355X the kernel reads the native row layout
    with 16-byte loads, so the bytes are uploaded unchanged."""

    def __init__(self, raw, type_name, K, N, bias=None):
        if type_name not in _NATIVE_TYPES:
            raise NotImplementedError("native ggml type %s" % type_name)
        self.type_name = type_name
        self.Kt, self.Nt = int(K), int(N)
        self.packed = ggml_transpose(raw, self.Nt, _row_bytes(type_name, self.Kt))
        self.bias = None if bias is None else (to_device(bias, torch.float32) if isinstance(bias, torch.Tensor)
                                               else to_device(np.asarray(bias, np.float32)))

    def forward(self, x, out_dtype=torch.float32):
        xt = as_activation(x)
        lead = xt.shape[:-1]
        of = ggml_matmul(xt.reshape(-1, self.Kt), self.packed, self.type_name, self.Kt, self.Nt,
                         bias=self.bias, out_dtype=out_dtype)
        return of.reshape(*lead, self.Nt)

    __call__ = forward

    def dequantize(self):
        """fp32 (N, K) weight, bit-exact with `ggufload.dequant` of the same bytes."""
        nb = self.Nt * (self.Kt // _NATIVE_TYPES[self.type_name][0])
        return ggml_dequant(self.packed, self.type_name, nb).reshape(self.Nt, self.Kt)

    def nbytes(self):
        return int(self.packed.numel() + (0 if self.bias is None else self.bias.numel() * 4))


# ---- sparse MoE ----------------------------------------------------------------------
def moe_route_bytes(T, E, k):
    n = ctypes.c_size_t(0)
    _lib.call("miq_moe_route_bytes", T, E, k, ctypes.byref(n))
    return int(n.value)


class MoEExperts:
    """The experts of one sparse-MoE layer, stacked on the device for the grouped kernels.

    `experts` is the reference's list of {"gate", "up", "down"} GPTQ linears
    (`webtorch/lm_engine.py:294-299`; built by `webtorch/llm.py:522-534`), here
    `QuantizedLinear` objects (or AutoGPTQ layer dicts) that share group size, bit width, zero
    offset and scale dtype. Calling it runs routing, gate/up, down and combine on the current
    stream with no host synchronisation."""

    def __init__(self, experts):
        self.native = all(isinstance(e[k], GGMLLinear) for e in experts for k in ("gate", "up", "down"))
        if self.native:
            self._init_native(experts)
            return
        exps = [{k: _as_linear(e[k]) for k in ("gate", "up", "down")} for e in experts]
        g0 = exps[0]["gate"]
        self.E = len(exps)
        self.H, self.I = g0.Kp, g0.Np
        self.gs, self.bits, self.zoff = g0.gs, g0.bits, g0.zero_offset
        for e in exps:
            for name, (K, N) in (("gate", (self.H, self.I)), ("up", (self.H, self.I)), ("down", (self.I, self.H))):
                q = e[name]
                if (q.Kp, q.Np, q.gs, q.bits, q.zero_offset) != (K, N, self.gs, self.bits, self.zoff):
                    raise ValueError("experts must share shapes, group size, bits and zero offset")
                if q.perm is not None:
                    raise NotImplementedError("act-order (g_idx) experts")
                if (q.Kt, q.Nt) != (q.Kp, q.Np):
                    raise NotImplementedError("expert linears stored padded (K %d of %d, N %d of %d)" % (
                        q.Kt, q.Kp, q.Nt, q.Np))
        self.sdt = exps[0]["gate"].scales.dtype
        self.w = {}
        for name in ("gate", "up", "down"):
            self.w[name] = tuple(torch.stack([getattr(e[name], a).to(self.sdt) if a == "scales" else getattr(e[name], a)
                                              for e in exps]).contiguous()
                                 for a in ("qweight", "qzeros", "scales"))
        # the experts' fp32 biases (`QuantizedLinear.forward` adds them to the product), stacked
        # [E][N] per projection; none when every bias is zero (the kernels then skip the adds)
        biased = any(bool(torch.any(e[n].bias != 0)) for e in exps for n in ("gate", "up", "down"))
        self.b = {n: torch.stack([e[n].bias for e in exps]).contiguous() if biased else None
                  for n in ("gate", "up", "down")}

    def _init_native(self, experts):
        """GGUF experts kept in their file encoding (`_gexperts` on the native path,
        `webtorch/llm.py:731-760`): each projection's experts stacked as [E][rows of blocks]; gate
        and up of one block type are stacked per expert as one (2I)-row matrix so one launch
        computes both."""
        self.E = len(experts)
        g0, d0 = experts[0]["gate"], experts[0]["down"]
        self.H, self.I = g0.Kt, g0.Nt
        for e in experts:
            for name, (K, N) in (("gate", (self.H, self.I)), ("up", (self.H, self.I)), ("down", (self.I, self.H))):
                q = e[name]
                if (q.Kt, q.Nt) != (K, N) or q.type_name != experts[0][name].type_name:
                    raise ValueError("experts must share shapes and block types per projection")
                if q.bias is not None:
                    raise NotImplementedError("GGUF expert linears with a bias")
                if q.type_name in DENSE_TYPES:
                    raise NotImplementedError("unquantized (%s) GGUF experts" % q.type_name)
        self.types = {n: experts[0][n].type_name for n in ("gate", "up", "down")}
        self.fused_gate_up = self.types["gate"] == self.types["up"]
        stack = lambda names: torch.stack([torch.cat([e[n].packed.reshape(-1) for n in names])  # noqa: E731
                                           for e in experts]).contiguous()
        if self.fused_gate_up:
            self.wb = {"gate_up": stack(("gate", "up"))}
        else:
            self.wb = {"gate": stack(("gate",)), "up": stack(("up",))}
        self.wb["down"] = stack(("down",))
        self.sdt = None

    def _block_native(self, xt, lg, k, norm_topk_prob, out):
        T = int(xt.shape[0])
        st = stream_handle()
        route = torch.empty(moe_route_bytes(T, self.E, k), dtype=torch.uint8, device=xt.device)
        gu = torch.empty((T * k, 2 * self.I), dtype=torch.float32, device=xt.device)
        h = torch.empty((T * k, self.I), dtype=torch.float32, device=xt.device)
        y = torch.empty((T * k, self.H), dtype=torch.float32, device=xt.device)
        _lib.call("miq_moe_route", ptr(lg), T, self.E, k, int(bool(norm_topk_prob)), ptr(route), route.numel(), st)

        def run(xin, gather, weighted, wb, tname, o, K, N):
            _lib.call("miq_moe_ggml_gemv", ptr(xin), dtype_code(xin), ptr(route), T, self.E, k, gather, weighted,
                      ptr(wb), _NATIVE_TYPES[tname][2], wb.shape[1], ptr(o), K, N, st)
        if self.fused_gate_up:
            run(xt, 1, 0, self.wb["gate_up"], self.types["gate"], gu, self.H, 2 * self.I)
        else:
            g, u = gu[:, :self.I], gu[:, self.I:]
            gtmp = torch.empty((T * k, self.I), dtype=torch.float32, device=xt.device)
            utmp = torch.empty((T * k, self.I), dtype=torch.float32, device=xt.device)
            run(xt, 1, 0, self.wb["gate"], self.types["gate"], gtmp, self.H, self.I)
            run(xt, 1, 0, self.wb["up"], self.types["up"], utmp, self.H, self.I)
            g.copy_(gtmp)
            u.copy_(utmp)
        _lib.call("miq_silu_mul", ptr(gu), ptr(h), T * k, self.I, st)
        run(h, 0, 1, self.wb["down"], self.types["down"], y, self.I, self.H)
        _lib.call("miq_moe_combine", ptr(y), ptr(route), T, self.E, k, ptr(out), self.H, st)
        self.last_route = route

    # tokens per routing pass: the router handles T * k <= MAX_ROUTED picks at a time
    MAX_ROUTED = 4096

    def __call__(self, x, logits, top_k, norm_topk_prob=True):
        """x (T, H) fp16 or fp32 -> (T, H) float32; logits (T, E) router outputs. fp32 x stays
        fp32 (it enters the matrix cores as row-scaled fp16 hi/lo planes); longer batches are
        routed in blocks of MAX_ROUTED // top_k tokens (tokens are independent)."""
        xt = as_activation(x)
        T = int(xt.shape[0])
        xt = aligned16(xt.reshape(T, self.H).contiguous())
        lg = as_activation(logits).float().reshape(T, self.E).contiguous()
        out = torch.empty((T, self.H), dtype=torch.float32, device=xt.device)
        k = int(top_k)
        step = max(1, self.MAX_ROUTED // k)
        for t0 in range(0, T, step):
            t1 = min(T, t0 + step)
            self._block(xt[t0:t1], lg[t0:t1], k, norm_topk_prob, out[t0:t1])
        return out

    def _block(self, xt, lg, k, norm_topk_prob, out):
        if self.native:
            return self._block_native(xt, lg, k, norm_topk_prob, out)
        T = int(xt.shape[0])
        route = torch.empty(moe_route_bytes(T, self.E, k), dtype=torch.uint8, device=xt.device)
        h = torch.empty((T * k, self.I), dtype=torch.float32, device=xt.device)
        y = torch.empty((T * k, self.H), dtype=torch.float32, device=xt.device)
        st = stream_handle()
        sd = dtype_code(self.w["gate"][2])
        xt = aligned16(xt)
        _lib.call("miq_moe_route", ptr(lg), T, self.E, k, int(bool(norm_topk_prob)), ptr(route), route.numel(), st)
        g, u, d = self.w["gate"], self.w["up"], self.w["down"]
        _lib.call("miq_moe_gate_up", ptr(xt), dtype_code(xt), ptr(route), T, self.E, k, ptr(g[0]), ptr(g[1]), ptr(g[2]),
                  ptr(u[0]), ptr(u[1]), ptr(u[2]), sd, ptr(self.b["gate"]), ptr(self.b["up"]), ptr(h), self.H, self.I,
                  self.gs, self.bits, float(self.zoff), st)
        _lib.call("miq_moe_down", ptr(h), ptr(route), T, self.E, k, ptr(d[0]), ptr(d[1]), ptr(d[2]), sd,
                  ptr(self.b["down"]), ptr(y), self.I, self.H, self.gs, self.bits, float(self.zoff), st)
        _lib.call("miq_moe_combine", ptr(y), ptr(route), T, self.E, k, ptr(out), self.H, st)
        self.last_route = route


class SharedExpert:
    """The optional always-on expert of a Qwen-style MoE layer with its sigmoid gate
    (`webtorch/lm_engine.py:322-328`): ys = down(silu(gate(x)) * up(x)) in fp32, times
    sigmoid(shared_gate(x)) if present, added to the routed output. gate and up run as one fused
    GEMM (their columns concatenated), SwiGLU and the gated add are kernels."""

    def __init__(self, shared, shared_gate=None):
        g, u, dn = (_as_linear(shared[n]) for n in ("gate", "up", "down"))
        if (g.Kp, g.Np, g.gs, g.bits, g.zero_offset) != (u.Kp, u.Np, u.gs, u.bits, u.zero_offset) or g.perm is not None:
            raise ValueError("shared gate and up must share shape, group size, bits and zero offset")
        sdt = torch.float32 if torch.float32 in (g.scales.dtype, u.scales.dtype) else g.scales.dtype
        self.gate_up = QuantizedLinear(torch.cat([g.qweight, u.qweight], 1), torch.cat([g.qzeros, u.qzeros], 1),
                                       torch.cat([g.scales.to(sdt), u.scales.to(sdt)], 1),
                                       torch.cat([g.bias, u.bias]), g.Kt, g.Nt + u.Nt, g.Kp, g.Np + u.Np, g.gs, g.bits,
                                       g.zero_offset)
        self.I = g.Np
        self.down = dn
        self.gate = None if shared_gate is None else _as_linear(shared_gate)

    def add_to(self, out, x):
        """out (T, H) fp32 += the gated shared-expert output for x (T, H)."""
        T = int(x.shape[0])
        gu = self.gate_up(x)                                   # (T, 2I) fp32
        act = torch.empty((T, self.I), dtype=torch.float32, device=gu.device)
        st = stream_handle()
        _lib.call("miq_silu_mul", ptr(gu), ptr(act), T, self.I, st)
        ys = self.down(act).contiguous()                       # (T, H) fp32
        gl = None if self.gate is None else self.gate(x).reshape(T).contiguous()
        _lib.call("miq_moe_shared_add", ptr(out), ptr(ys), ptr(gl), T, int(out.shape[1]), st)
        return out


def _as_linear(d):
    if isinstance(d, QuantizedLinear):
        return d
    return QuantizedLinear.from_autogptq(d["qweight"], d["qzeros"], d["scales"], d.get("bias"), d["gs"], d["bits"])


def moe_mlp(lm, lay, x):
    """Sparse MoE MLP, drop-in for `moe_mlp(lm, lay, x)` (`webtorch/lm_engine.py:294-329`) with
    the same `lay["moe"]` schema: gate (router linear), experts [{gate, up, down}], top_k,
    norm_topk_prob, shared {gate, up, down} | None, shared_gate | None. Routing runs on the
    device (the reference reads the router logits back to the host); the stacked experts (and
    the fused shared expert) are cached in the dict. fp32 activations stay fp32 throughout."""
    m = lay["moe"]
    xt = as_activation(x)
    T = int(xt.shape[0])
    logits = m["gate"](xt)
    ex = m.get("_grouped")
    if ex is None:
        ex = m["_grouped"] = MoEExperts(m["experts"])
    out = ex(xt, logits, m["top_k"], m.get("norm_topk_prob", True))
    if m.get("shared"):
        se = m.get("_shared")
        if se is None:
            se = m["_shared"] = SharedExpert(m["shared"], m.get("shared_gate"))
        se.add_to(out, xt.reshape(T, -1))
    return out
