"""GPTQ int4 decoder (Qwen2 family) on MI355X with a captured decode step: the drop-in
counterpart of the reference's `CausalLM` decode path (`webtorch/llm.py:506-647, 1258-1336,
1465-1489, 1558-1636, 1716-1817`) for GPTQ checkpoints.

Host code only plans and launches; every operator is a HIP kernel from libmiq.so. The
activations stay fp32, as in the reference's numpy decode. One decode step runs embedding ->
24 x (RMSNorm, fused q|k|v GEMV + bias, RoPE + KV write, causal GQA attention, o GEMV +
residual, RMSNorm, fused gate|up GEMV, SwiGLU, down GEMV + residual) -> final RMSNorm -> head
GEMV -> device argmax. The position and the token ids live in a device "decode state", so the
step is recorded once as a HIP graph and replayed per token with no host work in between (the
reference re-uploads inputs and reads the logits back to the host every token,
`webtorch/llm.py:1582-1589, 1808-1814`).

Where the shape allows it (`miq_decode_persistent_plan`), the one-token step is a single
persistent launch instead of 5 launches per layer: one workgroup per CU with a fixed role
(a 64-column tile of a projection, a query head, or a tile and K-slice of the down
projection); the workgroups exchange activations through tagged device-scope words, so the
step has no kernel boundary and each projection's weights are fetched a layer ahead.
`persistent=False` keeps the launch sequence; prefill always uses it. The persistent step needs
every workgroup resident at once: if other work on the GPU keeps one off its CU, the step's
bounded waits time out, it and the steps after it leave the decode state alone, and
`generate` finishes the sequence with the launch sequence (with a RuntimeWarning).

Layout choices: q, k and v (and gate and up) share their input, so their GPTQ tensors are
concatenated along the output dimension at load time and run as one GEMV (per-column groups
make this identical to separate layers). The tied head is re-quantized from the fp16
embedding on the device, bit-exact with `_gptq_quantize` (`webtorch/_core.py:3782-3824`;
per-column quantization makes the reference's 4096-row blocks, `llm.py:594-602`, one matrix).
"""
import ctypes
import math
import time
import warnings

import numpy as np
import torch

from . import _lib, core
from .core import ptr, stream_handle


class GenResult:
    """Result of `generate` (`webtorch/llm.py:273-279`)."""

    def __init__(self, text, tokens, ttft_s, decode_tok_s):
        self.text = text
        self.tokens = tokens
        self.ttft_s = ttft_s
        self.decode_tok_s = decode_tok_s

    def __repr__(self):
        return "GenResult(ttft=%.4fs, %.1f tok/s, %d tokens)" % (self.ttft_s, self.decode_tok_s, len(self.tokens))


def _cat_layers(parts, gs, bits):
    """Concatenate GPTQ layers that share K along the output dimension, on the device."""
    zoffs = {float(p.get("zoff", 1.0)) for p in parts}
    if len(zoffs) != 1:
        raise ValueError("fused projections must share their zero offset")
    cat = lambda key, dt=None: torch.cat([core.to_device(p[key], dt) for p in parts], dim=1)  # noqa: E731
    out = {"qweight": cat("qweight", torch.int32), "qzeros": cat("qzeros", torch.int32), "zoff": zoffs.pop()}
    sdt = {core.to_device(p["scales"]).dtype for p in parts}
    out["scales"] = cat("scales", torch.float32 if torch.float32 in sdt else None)
    if any(p.get("bias") is not None for p in parts):
        out["bias"] = torch.cat([core.to_device(p["bias"], torch.float32) if p.get("bias") is not None
                                 else torch.zeros(int(np.shape(p["qweight"])[1]), dtype=torch.float32,
                                                  device=core.device()) for p in parts])
    return out


def _gptq_dict(d, gs, bits):
    """A GPTQ layer dict as a QuantizedLinear with its own zero offset (AutoGPTQ tensors: 1)."""
    per = 32 // bits
    K, N = int(np.shape(d["qweight"])[0]) * per, int(np.shape(d["qweight"])[1])
    return core.QuantizedLinear(d["qweight"], d["qzeros"], d["scales"], d.get("bias"), d.get("Kt", K), d.get("Nt", N),
                                K, N, gs, bits, zero_offset=float(d.get("zoff", 1.0)))


class _Lin:
    """Device tensors of one (possibly fused) GPTQ linear. The zero offset is the layer's own:
    1 for AutoGPTQ tensors (stored zero - 1), 0 for layers quantized on load. K and N are the
    stored (padded) sizes; Kt and Nt the layer's own (a layer quantized on load pads K to the
    group multiple and N to the pack width: `padded` layers take Kt inputs and give Nt outputs)."""

    def __init__(self, d, K, gs, bits, zoff=None):
        self.qweight = core.to_device(d["qweight"], torch.int32)
        self.qzeros = core.to_device(d["qzeros"], torch.int32)
        self.scales = core.to_device(d["scales"])
        self.K, self.N = int(self.qweight.shape[0]) * (32 // bits), int(self.qweight.shape[1])
        self.Kt, self.Nt = int(d.get("Kt", self.K)), int(d.get("Nt", self.N))
        if self.Kt != K:
            raise ValueError("layer takes %d inputs where %d are expected" % (self.Kt, K))
        self.padded = (self.Kt, self.Nt) != (self.K, self.N)
        b = d.get("bias")
        self.bias = None
        if b is not None:
            bt = core.to_device(b, torch.float32).reshape(-1)
            self.bias = bt if bt.numel() == self.N else torch.nn.functional.pad(bt, (0, self.N - bt.numel()))
        self.gs, self.bits = gs, bits
        self.zoff = float(d.get("zoff", 1.0) if zoff is None else zoff)


def _lin_n(lin):
    return int(lin.Nt) if isinstance(lin, (core.GGMLLinear, _Lin)) else int(lin.N)


def _dict_padded(d, bits):
    """Does a GPTQ layer dict store more rows or columns than the layer has (quantize-on-load
    padding)?"""
    K, N = int(np.shape(d["qweight"])[0]) * (32 // bits), int(np.shape(d["qweight"])[1])
    return int(d.get("Kt", K)) != K or int(d.get("Nt", N)) != N


class _Group:
    """Linears that share their input and fill consecutive column ranges of one output: the
    q|k|v (or gate|up) of a GGUF layer whose tensors use different block types, so that their
    bytes cannot be concatenated into one matrix."""

    def __init__(self, parts):
        self.parts = parts
        self.N = sum(_lin_n(q) for q in parts)
        self.bias = None


def _fuse(parts, K, gs, bits):
    """One layer for projections that share K: GPTQ dicts concatenated along the output
    dimension; GGUF layers of one block type likewise (their rows are whole blocks); a mix as a
    _Group."""
    if all(isinstance(q, dict) for q in parts) and not any(_dict_padded(q, bits) for q in parts):
        return _Lin(_cat_layers(parts, gs, bits), K, gs, bits)
    lins = [q if isinstance(q, core.GGMLLinear) else _Lin(q, K, gs, bits) for q in parts]
    # adjacent GGUF layers of one block type become one layer (q and k of a Q4_K_M file's layer
    # whose v is Q6_K: two launches instead of three)
    runs = []
    for q in lins:
        if runs and isinstance(q, core.GGMLLinear) and isinstance(runs[-1][-1], core.GGMLLinear) and \
                q.type_name == runs[-1][-1].type_name:
            runs[-1].append(q)
        else:
            runs.append([q])
    merged = [_cat_ggml(r, K) if len(r) > 1 else r[0] for r in runs]
    return merged[0] if len(merged) == 1 else _Group(merged)


def _cat_ggml(lins, K):
    """GGUF layers of one block type and input width as one layer (rows are whole blocks)."""
    N = sum(q.Nt for q in lins)
    bias = None
    if any(q.bias is not None for q in lins):
        bias = torch.cat([q.bias if q.bias is not None else torch.zeros(q.Nt, device=core.device()) for q in lins])
    return core.GGMLLinear(torch.cat([q.packed for q in lins]), lins[0].type_name, K, N, bias)


def _mk_lin(d, K, gs, bits):
    return d if isinstance(d, core.GGMLLinear) else _Lin(d, K, gs, bits)


def _interleave_gate_up(gu, I):
    """The fused [gate | up] GPTQ tensors with their columns regrouped by 64: gate columns
    32 t .. 32 t + 31, then up columns 32 t .. 32 t + 31, for t = 0 .. I / 32 - 1, so that one
    64-column tile of the persistent step holds matching gate and up columns. A column
    permutation: qweight and scales gather columns, qzeros (8 columns per word at int4) whole
    words of 4."""
    dev = gu.qweight.device
    cols = torch.arange(2 * I, device=dev).view(2, I // 32, 32).permute(1, 0, 2).reshape(-1)
    words = torch.arange(2 * I // 8, device=dev).view(2, I // 32, 4).permute(1, 0, 2).reshape(-1)
    return (gu.qweight[:, cols].contiguous(), gu.qzeros[:, words].contiguous(), gu.scales[:, cols].contiguous())


class CausalLM:
    """Qwen2-shaped GPTQ decoder with device-resident decode (see module docstring).

    Build with `CausalLM.from_weights(weights, lmax)` where `weights` holds AutoGPTQ tensors per
    layer ({"q","k","v","o","gate","up","down"} dicts with qweight/qzeros/scales[/bias],
    "in_ln", "post_ln"), the fp16 "embed" table, optionally an fp16 "head" (V, H) for an untied
    model (else the head is tied to the embedding), "final_norm" and "cfg"
    (L, H, NH, NKV, HD, I, V, gs, bits[, eps, theta]); or with `CausalLM.from_gptq(path)` from an
    AutoGPTQ safetensors directory."""

    def __init__(self, weights, lmax=256, fused=True, persistent=None):
        c = weights["cfg"]
        # decode tokens per captured graph: a replay costs ~5 us more than a plain launch of the
        # same kernel, so one graph holds several one-token steps (348.5 against 351.7 us per token
        # for the persistent step of the Qwen2-0.5B shape, eager launches 346.7 us)
        self.graph_tokens = 16
        self.fused = bool(fused)  # one-token steps use the fused launches (else the prefill path)
        self.persistent = persistent  # None: the persistent step where the shape allows it
        self.L, self.H, self.NH, self.NKV, self.HD = c["L"], c["H"], c["NH"], c["NKV"], c["HD"]
        self.I, self.V, self.gs, self.bits = c["I"], c["V"], c["gs"], c["bits"]
        self.eps = float(c.get("eps", 1e-6))
        self.theta = float(c.get("theta", 1e6))
        self.lmax = int(lmax)
        core.device()
        self.layers = []
        vec = lambda v: None if v is None else core.to_device(v if isinstance(v, torch.Tensor) else  # noqa: E731
                                                              np.asarray(v, np.float32), torch.float32)
        for lay in weights["layers"]:
            d = {"qkv": _fuse([lay["q"], lay["k"], lay["v"]], self.H, self.gs, self.bits),
                 "o": _mk_lin(lay["o"], self.NH * self.HD, self.gs, self.bits),
                 "in_ln": vec(lay["in_ln"]), "post_ln": vec(lay["post_ln"]),
                 "qn": vec(lay.get("qn")), "kn": vec(lay.get("kn"))}
            mo = lay.get("moe")
            if mo:  # sparse MoE MLP (`CausalLM._mlp` -> `moe_mlp`, `webtorch/llm.py:1489-1496`)
                lin = lambda e: e if isinstance(e, core.GGMLLinear) else _gptq_dict(e, self.gs, self.bits)  # noqa: E731
                d["moe"] = {"router": _mk_lin(mo["router"], self.H, self.gs, self.bits),
                            "experts": core.MoEExperts([{k: lin(e[k]) for k in ("gate", "up", "down")}
                                                        for e in mo["experts"]]),
                            "top_k": int(mo["top_k"]),
                            "shared": core.SharedExpert({k: lin(mo["shared"][k]) for k in ("gate", "up", "down")},
                                                        mo.get("shared_gate")) if mo.get("shared") else None}
            else:
                d["gate_up"] = _fuse([lay["gate"], lay["up"]], self.H, self.gs, self.bits)
                d["down"] = _mk_lin(lay["down"], self.I, self.gs, self.bits)
            self.layers.append(d)
        self.has_moe = any("moe" in lay for lay in self.layers)
        self.has_qk_norm = any(lay["qn"] is not None or lay["kn"] is not None for lay in self.layers)
        emb = weights["embed"]
        if isinstance(emb, torch.Tensor) and emb.dtype == torch.float32:
            self.embed = core.to_device(emb)  # a GGUF token_embd decoded to exact fp32
        else:
            self.embed = core.to_device(np.asarray(emb, np.float16))
        self.final_norm = core.to_device(weights["final_norm"], torch.float32) if isinstance(
            weights["final_norm"], torch.Tensor) else core.to_device(np.asarray(weights["final_norm"], np.float32))
        if weights.get("head_linear") is not None:  # a GGUF head: native, or already quantized
            self.head = _mk_lin(weights["head_linear"], self.H, self.gs, self.bits)
        else:
            head = weights.get("head")
            if head is not None and tuple(np.shape(head)) != (self.V, self.H):
                raise ValueError("head must be (V, H) = (%d, %d), got %s" % (self.V, self.H, np.shape(head)))
            self.head = self._quantize_head(None if head is None else core.to_device(np.asarray(head, np.float16)))
        # layers kept in a GGUF block encoding run the unfused launch sequence (the fused and
        # persistent one-token kernels read GPTQ tensors)
        lins = [self.head] + [lay[k] for lay in self.layers for k in ("qkv", "o", "gate_up", "down") if k in lay]
        lins += [lay["moe"]["router"] for lay in self.layers if "moe" in lay]
        parts = [p for q in lins for p in (q.parts if isinstance(q, _Group) else [q])]
        self.native_gguf = any(isinstance(p, core.GGMLLinear) for p in parts)
        # the fused one-token kernels (RMSNorm / SwiGLU staging, persistent step) read K inputs and
        # write N outputs: layers stored padded run the launch sequence
        self.padded = any(getattr(p, "padded", False) for p in parts)
        if self.native_gguf or self.padded:
            self.fused = False
        self._alloc()
        self._graphs = {}  # decode tokens -> captured graph of them
        self.fallback_steps = 0  # tokens of the last generate() that a timed-out persistent step left

    @classmethod
    def from_weights(cls, weights, lmax=256, fused=True, persistent=None):
        return cls(weights, lmax, fused, persistent)

    @classmethod
    def from_gptq(cls, path, lmax=None, fused=True, persistent=None):
        """Load an AutoGPTQ safetensors directory (config.json + model.safetensors or an index
        and shards), as the reference's `from_gptq` does (`webtorch/llm.py:614-647`). `lmax=None`
        takes the model's declared context, capped by a 2 GiB KV-cache budget."""
        from . import checkpoint
        w, declared = checkpoint.gptq_weights(path)
        c = w["cfg"]
        return cls(w, checkpoint.auto_lmax(lmax, declared, c["L"], c["NKV"], c["HD"]), fused, persistent)

    @classmethod
    def from_fp16(cls, path, lmax=None, quantize=None, fused=True, persistent=None):
        """Load a plain fp16/bf16 HuggingFace safetensors directory, quantizing every linear to
        int`quantize` (4 or 8) on the device as it loads (`webtorch/llm.py:1221-1257`: group
        size 128, zero offset 0, fp32 scales; the tied head as `_quantize_head`). Unquantized
        fp16 execution (`quantize=None` in the reference) is not part of this library."""
        if quantize is None:
            raise NotImplementedError("unquantized fp16 execution is not part of this library: "
                                      "pass quantize=4 or quantize=8 (dtype='int4' / 'int8')")
        from . import checkpoint
        w, declared = checkpoint.fp16_weights(path, int(quantize))
        c = w["cfg"]
        return cls(w, checkpoint.auto_lmax(lmax, declared, c["L"], c["NKV"], c["HD"]), fused, persistent)

    @classmethod
    def from_gguf(cls, path, lmax=None, bits=None, weights="native", persistent=None):
        """Load a llama.cpp GGUF decoder (`CausalLM.from_gguf`, `webtorch/llm.py:856-1129`).
        `weights="native"` (the default) keeps every weight whose block type has a kernel here
        in the file's own encoding and runs the unfused launch sequence; "requant" decodes each
        weight on the device and quantizes it to int`bits` (the file's own width when None),
        which runs the fused GPTQ path. `lmax=None` takes the context length the file declares,
        capped by the KV-cache budget."""
        from . import checkpoint
        w, declared = checkpoint.gguf_weights(path, bits, weights)
        c = w["cfg"]
        return cls(w, checkpoint.auto_lmax(lmax, declared, c["L"], c["NKV"], c["HD"]), True, persistent)

    # ---- load-time ----
    def _quantize_head(self, head=None):
        """The head (the fp16 embedding when tied, else the model's fp16 (V, H) head) quantized
        on the device to int4 GPTQ with fp32 scales and zero offset 0, as `_quantize_head` does
        (`webtorch/llm.py:594-612`)."""
        qw, qz, sc, K, N = core.gptq_quantize(self.embed if head is None else head, self.gs, self.bits,
                                              from_out_in=True)
        return _Lin({"qweight": qw, "qzeros": qz, "scales": sc}, K, self.gs, self.bits, 0.0)

    def _alloc(self):
        dev, f32, T = core.device(), torch.float32, self.lmax
        z = lambda *s: torch.zeros(s, dtype=f32, device=dev)  # noqa: E731
        qkvd = (self.NH + 2 * self.NKV) * self.HD
        self.buf = {"h": z(T, self.H), "xn": z(T, self.H), "qkv": z(T, qkvd), "q": z(T, self.NH * self.HD),
                    "att": z(T, self.NH * self.HD), "tmp": z(T, self.H), "hl": z(1, self.H), "logits": z(1, self.V)}
        if not all("moe" in lay for lay in self.layers):
            self.buf.update(gu=z(T, 2 * self.I), act=z(T, self.I))
        if self.has_moe:
            E = max(_lin_n(lay["moe"]["router"]) for lay in self.layers if "moe" in lay)
            self.buf["rlog"] = z(T, E)
        self.kc = torch.zeros((self.L, self.NKV, self.lmax, self.HD), dtype=f32, device=dev)
        self.vc = torch.zeros_like(self.kc)
        # RoPE tables exactly as `_rope_np` builds them (float64 angles, rounded once to fp32)
        inv = 1.0 / (self.theta ** (np.arange(0, self.HD, 2, dtype=np.float64) / self.HD))
        ang = np.arange(0, T, dtype=np.float64)[:, None] * inv[None, :]
        self.cos_t = core.to_device(np.cos(ang).astype(np.float32))
        self.sin_t = core.to_device(np.sin(ang).astype(np.float32))
        self.ids = torch.zeros(T, dtype=torch.int32, device=dev)
        self.history = torch.zeros(T, dtype=torch.int32, device=dev)
        self.state = torch.zeros(_lib.lib().miq_decode_state_words(), dtype=torch.int32, device=dev)
        # one split-K workspace sized for every projection at T = 1 and at the largest prefill
        # (the need is not monotonic in the row count: wide enough layers stop splitting K)
        need = 0
        if isinstance(self.head, _Lin):
            need = core.gemv_workspace_bytes(1, self.head.K, self.head.N, self.gs, self.bits, _lib.MIQ_F32)
        lins = {}
        for lay in self.layers:
            for k in ("qkv", "o", "gate_up", "down"):
                if k in lay:
                    for i, q in enumerate(lay[k].parts if isinstance(lay[k], _Group) else [lay[k]]):
                        lins[(k, i)] = q
            if "moe" in lay:
                lins["router"] = lay["moe"]["router"]
        lins = {k: q for k, q in lins.items() if isinstance(q, _Lin)}  # GGUF kernels need no workspace
        for M in range(1, T + 1):  # the head only ever sees the last token
            for lin in lins.values():
                need = max(need, core.gemv_workspace_bytes(M, lin.K, lin.N, lin.gs, lin.bits, _lib.MIQ_F32))
                if M > core.GEMV_MAX_M:  # prefill rows on the matrix cores
                    need = max(need, core.gemm_f32x_workspace_bytes(M, lin.K, lin.N, lin.gs, lin.bits))
        self.ws = torch.zeros(max(need, 1 << 20), dtype=torch.uint8, device=dev)
        self._alloc_persistent()

    def _alloc_persistent(self):
        """Layer address table and exchange workspace of the persistent one-token step, if the
        shape is supported and the layers carry fp16 scales (else the launch sequence runs)."""
        self.pws = None
        if self.persistent is False or not self.fused:
            return
        if self.has_moe or self.has_qk_norm:
            if self.persistent:
                raise ValueError("the persistent decode step covers dense layers without QK-norm")
            return
        lays = self.layers
        lins = [lay[k] for lay in lays for k in ("qkv", "o", "gate_up", "down")]
        fp16 = all(q.scales.dtype == torch.float16 for q in lins)
        one_zoff = len({q.zoff for q in lins}) == 1
        if not fp16 or not one_zoff or self.head.scales.dtype != torch.float32:
            if self.persistent:
                raise ValueError("persistent decode needs fp16 layer scales, one zero offset and an fp32-scaled head")
            return
        grid, wsb = ctypes.c_int(0), ctypes.c_size_t(0)
        rc = _lib.lib().miq_decode_persistent_plan(self.L, self.H, self.NH, self.NKV, self.HD, self.I, self.V,
                                                   self.lmax, self.gs, self.bits, ctypes.byref(grid),
                                                   ctypes.byref(wsb))
        if rc != 0:
            if self.persistent:
                raise _lib.ERRORS.get(rc, _lib.MiqError)(
                    "persistent decode: %s" % _lib.lib().miq_last_error().decode(errors="replace"))
            return
        def a(t):
            return 0 if t is None else int(t.data_ptr())
        table = []
        self._gu_interleaved = []  # the persistent step's copies of gate|up (held for the table)
        for i, lay in enumerate(lays):
            qkv, o, gu, dn = lay["qkv"], lay["o"], lay["gate_up"], lay["down"]
            gi = _interleave_gate_up(gu, self.I)
            self._gu_interleaved.append(gi)
            table.append([a(qkv.qweight), a(qkv.qzeros), a(qkv.scales), a(qkv.bias),
                          a(o.qweight), a(o.qzeros), a(o.scales),
                          a(gi[0]), a(gi[1]), a(gi[2]),
                          a(dn.qweight), a(dn.qzeros), a(dn.scales),
                          a(lay["in_ln"]), a(lay["post_ln"]), a(self.kc[i]), a(self.vc[i]), 0, 0, 0])
        self.layer_table = torch.tensor(table, dtype=torch.int64, device=core.device())
        self.pws = torch.zeros(int(wsb.value), dtype=torch.uint8, device=core.device())
        self.persistent_grid = int(grid.value)

    def persistent_error(self):
        """Error bits of the persistent step's last runs (0 if none; see miq.h)."""
        if self.pws is None:
            return 0
        return int(self.pws[4:8].view(torch.int32).item())

    # ---- one forward over T tokens at the device position ----
    def _linear(self, lin, x, out, bias=None):
        if isinstance(lin, core.GGMLLinear):
            core.ggml_matmul(x, lin.packed, lin.type_name, lin.Kt, lin.Nt, bias=lin.bias if bias is None else bias,
                             out=out)
        elif isinstance(lin, _Group):
            # part outputs land in column ranges: directly for one row (the range is contiguous),
            # through a temporary for more
            c0, M = 0, int(x.shape[0])
            for part in lin.parts:
                n = _lin_n(part)
                if M == 1:
                    self._linear(part, x, out[:, c0:c0 + n])
                else:
                    tmp = torch.empty((M, n), dtype=out.dtype, device=out.device)
                    self._linear(part, x, tmp)
                    out[:, c0:c0 + n].copy_(tmp)
                c0 += n
        elif lin.padded:
            # the reference's QuantizedLinear.forward: x zero-padded to Kp, the output sliced to Nt
            # (`webtorch/_core.py:4446-4456`)
            xp = x if lin.Kt == lin.K else torch.nn.functional.pad(x, (0, lin.K - lin.Kt))
            tmp = torch.empty((int(x.shape[0]), lin.N), dtype=out.dtype, device=out.device)
            core._gptq_matmul(xp.contiguous(), lin.qweight, lin.qzeros, lin.scales, lin.K, lin.N, lin.gs, lin.bits,
                              lin.zoff, bias=lin.bias, out=tmp, ws=self.ws)
            if bias is not None:
                raise ValueError("a padded layer takes no bias override (its residual adds separately)")
            out.copy_(tmp[:, :lin.Nt])
        else:
            core._gptq_matmul(x, lin.qweight, lin.qzeros, lin.scales, lin.K, lin.N, lin.gs, lin.bits, lin.zoff,
                              bias=lin.bias if bias is None else bias, out=out, ws=self.ws)

    def _embed(self, T):
        if self.embed.dtype == torch.float32:
            _lib.call("miq_embed_f32", ptr(self.ids), ptr(self.embed), ptr(self.buf["h"]), T, self.H, self.V,
                      stream_handle())
        else:
            _lib.call("miq_embed", ptr(self.ids), ptr(self.embed), ptr(self.buf["h"]), T, self.H, self.V,
                      stream_handle())

    def _fused(self, lin, x, mode, norm_w, out, bias=None):
        """One-token GEMV with RMSNorm (mode 1) or SwiGLU (mode 2) applied to x while staging."""
        _lib.call("miq_gptq_gemv_fused", ptr(x), mode, ptr(norm_w), self.eps, None, ptr(lin.qweight),
                  ptr(lin.qzeros), ptr(lin.scales), core.dtype_code(lin.scales), ptr(lin.bias if bias is None else bias),
                  ptr(out), 1, lin.K, lin.N, lin.gs, lin.bits, float(lin.zoff), ptr(self.ws), self.ws.numel(),
                  stream_handle())

    def _decode_step(self):
        """One token at position state[0] (`_decode_fwd`, `webtorch/llm.py:1591-1616`): one
        persistent launch, or five launches per layer -- RMSNorm+qkv, RoPE+KV write+attention,
        o+residual, RMSNorm+gate|up, SwiGLU+down+residual -- then RMSNorm+head and the device
        argmax."""
        b, st = self.buf, stream_handle()
        if self.pws is not None:
            _lib.call("miq_decode_persistent", ptr(self.layer_table), ptr(self.embed), ptr(self.head.qweight),
                      ptr(self.head.qzeros), ptr(self.head.scales), ptr(self.final_norm), ptr(self.cos_t),
                      ptr(self.sin_t), ptr(self.ids), ptr(self.history), self.lmax, ptr(self.state),
                      ptr(b["logits"]), ptr(self.pws), self.pws.numel(), self.L, self.H, self.NH, self.NKV, self.HD,
                      self.I, self.V, self.lmax, self.gs, self.bits, self.eps, float(self.layers[0]["qkv"].zoff),
                      float(self.head.zoff), st)
            return
        h = b["h"][:1]
        self._embed(1)
        scale = 1.0 / math.sqrt(self.HD)
        for i, lay in enumerate(self.layers):
            self._fused(lay["qkv"], h, _lib.MIQ_X_RMSNORM, lay["in_ln"], b["qkv"])
            self._qk_norm(lay, 1)
            _lib.call("miq_attention_decode", ptr(b["qkv"]), ptr(self.state), ptr(self.cos_t), ptr(self.sin_t),
                      ptr(self.kc[i]), ptr(self.vc[i]), ptr(b["att"]), self.NH, self.NKV, self.HD, self.lmax, scale, st)
            self._linear(lay["o"], b["att"][:1], h, bias=h)
            if "moe" in lay:
                self._moe(lay, h, 1)
                continue
            self._fused(lay["gate_up"], h, _lib.MIQ_X_RMSNORM, lay["post_ln"], b["gu"])
            self._fused(lay["down"], b["gu"][:1], _lib.MIQ_X_SWIGLU, None, h, bias=h)
        self._fused(self.head, h, _lib.MIQ_X_RMSNORM, self.final_norm, b["logits"])
        _lib.call("miq_argmax_advance", ptr(b["logits"]), self.V, ptr(self.ids), ptr(self.history), self.lmax,
                  ptr(self.state), 1, st)

    def _step(self, T):
        """T tokens (ids[:T]) at positions state[0].. -> next token on the device
        (`_kv_forward`, `webtorch/llm.py:1619-1636`)."""
        if T == 1 and self.fused:
            return self._decode_step()
        b, st = self.buf, stream_handle()
        H, NH, NKV, HD, I = self.H, self.NH, self.NKV, self.HD, self.I
        h, xn = b["h"][:T], b["xn"][:T]
        self._embed(T)
        scale = 1.0 / math.sqrt(HD)
        for i, lay in enumerate(self.layers):
            _lib.call("miq_rmsnorm", ptr(h), ptr(lay["in_ln"]), ptr(xn), T, H, self.eps, st)
            self._linear(lay["qkv"], xn, b["qkv"][:T])
            self._qk_norm(lay, T)
            _lib.call("miq_rope_kv", ptr(b["qkv"]), ptr(self.state), ptr(self.cos_t), ptr(self.sin_t), ptr(b["q"]),
                      ptr(self.kc[i]), ptr(self.vc[i]), T, NH, NKV, HD, self.lmax, st)
            _lib.call("miq_attention", ptr(b["q"]), ptr(self.kc[i]), ptr(self.vc[i]), ptr(self.state), ptr(b["att"]), T,
                      NH, NKV, HD, self.lmax, scale, st)
            self._residual(lay["o"], b["att"][:T], h, T)
            if "moe" in lay:
                self._moe(lay, h, T)
                continue
            _lib.call("miq_rmsnorm", ptr(h), ptr(lay["post_ln"]), ptr(xn), T, H, self.eps, st)
            self._linear(lay["gate_up"], xn, b["gu"][:T])
            _lib.call("miq_silu_mul", ptr(b["gu"]), ptr(b["act"]), T, I, st)
            self._residual(lay["down"], b["act"][:T], h, T)
        _lib.call("miq_rmsnorm", ptr(h[T - 1:T]), ptr(self.final_norm), ptr(b["hl"]), 1, H, self.eps, st)
        self._linear(self.head, b["hl"], b["logits"])
        _lib.call("miq_argmax_advance", ptr(b["logits"]), self.V, ptr(self.ids), ptr(self.history), self.lmax,
                  ptr(self.state), T, st)

    def _qk_norm(self, lay, T):
        """Per-head RMSNorm of q and k in the fused q|k|v rows, before RoPE (Qwen3's QK-norm,
        `CausalLM._qkv`, `webtorch/llm.py:1498-1519`); nothing for layers without it."""
        if lay["qn"] is None and lay["kn"] is None:
            return
        _lib.call("miq_head_rmsnorm", ptr(self.buf["qkv"]), ptr(lay["qn"]), ptr(lay["kn"]), T, self.NH, self.NKV,
                  self.HD, self.eps, stream_handle())

    def _moe(self, lay, h, T):
        """h += the sparse-MoE MLP of RMSNorm(h) (`moe_mlp`, `webtorch/lm_engine.py:294-329`): router
        GEMV, device routing, grouped expert GEMMs and combine, plus the shared expert; all on the
        current stream, so the decode step stays capturable with live routing. The reference's
        layer dict names the flag "norm_topk" where `moe_mlp` reads "norm_topk_prob", so its top-k
        weights are always renormalised; so are these."""
        b, st = self.buf, stream_handle()
        mo = lay["moe"]
        xn = b["xn"][:T]
        _lib.call("miq_rmsnorm", ptr(h), ptr(lay["post_ln"]), ptr(xn), T, self.H, self.eps, st)
        E = _lin_n(mo["router"])
        logits = b["rlog"][:T, :E] if b["rlog"].shape[1] == E else b["rlog"].view(-1)[:T * E].view(T, E)
        self._linear(mo["router"], xn, logits)
        out = mo["experts"](xn, logits, mo["top_k"], True)
        if mo["shared"] is not None:
            mo["shared"].add_to(out, xn)
        _lib.call("miq_add", ptr(h), ptr(out), T * self.H, st)

    def _residual(self, lin, x, h, T):
        """h += x @ W: fused into the GEMV (bias = out = h) for one token, an add otherwise."""
        if T == 1 and lin.bias is None and not getattr(lin, "padded", False):
            self._linear(lin, x, h, bias=h)
        else:
            tmp = self.buf["tmp"][:T]
            self._linear(lin, x, tmp)
            _lib.call("miq_add", ptr(h), ptr(tmp), T * self.H, stream_handle())

    # ---- capture-replay ----
    def capture(self, tokens=1):
        """Record `tokens` decode steps (T = 1 each) as one HIP graph (`beginCapture`/`endCapture`,
        `webgpu/wgpy_backends/webgpu/platform.py:45-56`). Nothing in it depends on the host.
        First-use checks read results back, so they are skipped under capture: the one-row check
        of every GPTQ product class the step can run (bits, group size, scale dtype, zero offset)
        runs here, eagerly, first."""
        lins = [self.head] + [lay[k] for lay in self.layers for k in ("qkv", "o", "gate_up", "down") if k in lay]
        lins += [lay["moe"]["router"] for lay in self.layers if "moe" in lay]
        for q in {(p.bits, p.gs, p.scales.dtype, p.zoff): p for q in lins
                  for p in (q.parts if isinstance(q, _Group) else [q]) if isinstance(p, _Lin)}:
            core.selfcheck_gptq(1, torch.float32, *q)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(tokens):
                self._step(1)
        self._graphs[tokens] = g
        return g

    def graph(self, tokens):
        """The captured graph of `tokens` decode tokens, recorded on first use."""
        g = self._graphs.get(tokens)
        return g if g is not None else self.capture(tokens)

    def _chunks(self, n):
        """n decode tokens as (tokens per replay, replays): full graphs of `graph_tokens`, then one
        of the remainder."""
        full, rest = divmod(n, self.graph_tokens)
        return [(t, r) for t, r in ((self.graph_tokens, full), (rest, 1)) if t and r]

    def replay_tokens(self, n):
        """n decode tokens by graph replays (graphs recorded on first use)."""
        for t, r in self._chunks(n):
            g = self.graph(t)
            for _ in range(r):
                g.replay()

    def reset(self):
        self.state.zero_()
        self.history.zero_()
        if self.pws is not None:
            self.pws.zero_()  # epoch and every exchange tag back to zero (never a valid tag)

    def _plan_length(self, n_prompt, max_new):
        """Refuse sequences that do not fit the KV cache (`webtorch/llm.py:1397-1429`)."""
        if n_prompt < 1 or max_new < 1:
            raise ValueError("need at least one prompt token and one new token")
        if n_prompt + max_new > self.lmax:
            raise ValueError("prompt (%d) + max_new (%d) exceeds lmax %d" % (n_prompt, max_new, self.lmax))

    def _finish_after_timeout(self, max_new):
        """After the steps of a sequence: if a persistent step timed out waiting (it shared the
        GPU with other work, so its workgroups were not all resident), that step and every later
        one left the decode state alone; reset the exchange workspace and run the remaining
        tokens as the launch sequence. Returns how many tokens took that path."""
        err = self.persistent_error()
        if not err:
            return 0
        if err & 2:
            raise _lib.MiqError("persistent decode step failed (error bits %d): position past the KV cache" % err)
        left = max_new - int(self.state[1].item())
        warnings.warn("persistent decode step timed out waiting (another kernel on the GPU?); the remaining %d "
                      "token(s) run as the launch sequence" % left, RuntimeWarning, stacklevel=3)
        pws, self.pws = self.pws, None
        try:
            pws.zero_()
            for _ in range(left):
                self._step(1)
            torch.cuda.synchronize()
        finally:
            self.pws = pws
        return left

    def generate(self, ids, max_new, use_graph=True):
        """Greedy decode with no end token (`webtorch/llm.py:1716-1817` with do_sample off):
        prefill the prompt, then max_new - 1 decode steps. Returns a GenResult whose `tokens`
        are the max_new generated ids."""
        ids = [int(i) for i in ids]
        self._plan_length(len(ids), max_new)
        self.reset()
        self.ids[:len(ids)].copy_(torch.tensor(ids, dtype=torch.int32))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        self._step(len(ids))
        torch.cuda.synchronize()
        ttft = time.perf_counter() - t0
        chunks = self._chunks(max_new - 1)
        if use_graph:
            for t, _ in chunks:
                self.graph(t)
        t1 = time.perf_counter()
        if use_graph:
            for t, r in chunks:
                for _ in range(r):
                    self._graphs[t].replay()
        else:
            for _ in range(max_new - 1):
                self._step(1)
        torch.cuda.synchronize()
        self.fallback_steps = self._finish_after_timeout(max_new)
        dt = time.perf_counter() - t1
        toks = [int(t) for t in self.history[:max_new].cpu().numpy()]
        rate = (max_new - 1) / dt if max_new > 1 and dt > 0 else 0.0
        return GenResult("", toks, ttft, rate)


class AutoModelForCausalLM:
    """Entry point with the reference SDK's signature (`webtorch/_sdk.py:72-115`)."""

    @staticmethod
    def from_pretrained(path, dtype="auto", bits=None, lmax=None, weights="native"):
        """Load a decoder for the quantized engine, dispatching on `dtype` as the reference does
        (`AutoModelForCausalLM._load_raw`, `webtorch/_sdk.py:98-115`):

        * a directory whose config.json has `quantization_config` (AutoGPTQ int4/int8) loads at
          its own stored bits whatever `dtype` says (`from_gptq`);
        * a plain fp16/bf16 directory with dtype "int4" / "int8" is quantized on load
          (`from_fp16(quantize=4|8)`: group size 128, asymmetric, zero offset 0);
        * a `.gguf` file loads through `from_gguf` ("auto" keeps the width the file stores,
          "int4" / "int8" requantize, `bits` overrides, `weights` as in the reference).

        Unquantized execution ("fp16", or "auto" on a plain fp16 directory) is not part of this
        library and raises NotImplementedError. Unlike the reference this call is synchronous
        and does not cache loaded models."""
        p = str(path).rstrip("/")
        if dtype not in ("auto", "fp16", "int4", "int8"):
            raise ValueError("dtype must be 'auto', 'fp16', 'int4' or 'int8', got %r" % (dtype,))
        if p.endswith(".gguf"):
            if dtype == "fp16":
                raise NotImplementedError("unquantized fp16 execution is not part of this library")
            gb = 8 if dtype == "int8" else (4 if dtype == "int4" else bits)
            return CausalLM.from_gguf(p, lmax=lmax, bits=gb, weights=weights)
        from . import checkpoint
        if checkpoint.is_quantized_dir(p):
            return CausalLM.from_gptq(p, lmax=lmax)
        q = {"int4": 4, "int8": 8}.get(dtype)
        return CausalLM.from_fp16(p, lmax=lmax, quantize=q)
