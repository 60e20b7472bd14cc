"""On-disk checkpoints for the quantized-linear path: AutoGPTQ safetensors directories and the
GGUF container with native Q4_K upload.

* `SafetensorsDir` reads a HuggingFace model directory (`model.safetensors.index.json` and its
  shards, or a single `model.safetensors`) by byte ranges, as the reference's `_hdr` / `_np` /
  `_f16_chunked` do (`webtorch/llm.py:541-592`): an 8-byte little-endian header length, a
  JSON header (`__metadata__` dropped), tensors at `data_offsets` past the header. BF16 and
  F16 become fp32 and I32 stays int32 on `array`; `rows_f16` streams a 2-D table in row blocks
  straight to fp16, never holding the fp32 copy.
* `fp16_weights(path, bits)` builds it from a plain fp16/bf16 directory, quantizing every
  projection on the device on load (`from_fp16(quantize=4|8)`, `webtorch/llm.py:1211-1257`).
* `gptq_weights(path)` builds the weights dictionary of `llm.CausalLM` from an AutoGPTQ
  directory (`webtorch/llm.py:418-475, 506-539, 569-573, 614-647` -- `from_gptq`): the shape from
  `config.json`, AutoGPTQ tensors per projection, norms, the fp16 embedding and, for an untied
  model, the fp16 `lm_head.weight` (quantized on the device like the tied head). Scales stay in
  their fp16 file encoding (the reference widens them to fp32 on the host, an exact
  conversion); `g_idx` is not read, as in the reference (`_qlin` passes no g_idx).
* `parse_header` / `GGUFFile` read the GGUF container (`webtorch/ggufload.py:16-112`): magic,
  version, typed metadata, tensor infos (ggml dimension order, innermost first), data section
  aligned to `general.alignment`. `GGUFFile.linear` uploads a 2-D tensor unchanged as a
  `GGMLLinear` when a native kernel decodes its type (`_gload_native`,
  `webtorch/llm.py:762-783`) and returns None otherwise, for the caller to convert.

File formats are kept exactly (they are formats); the code is this package's own.
"""
import json
import os
import struct

import numpy as np

from . import core

# ---------------------------------------------------------------------------------------------
# safetensors


class SafetensorsDir:
    """Tensors of a HuggingFace safetensors model directory, read by byte range."""

    def __init__(self, path):
        self.base = str(path)
        self._hdrs = {}
        idx = os.path.join(self.base, "model.safetensors.index.json")
        if os.path.exists(idx):
            with open(idx) as f:
                self.index = dict(json.load(f)["weight_map"])
        else:
            h, _ = self.header("model.safetensors")
            self.index = {k: "model.safetensors" for k in h}

    def header(self, shard):
        """(tensor table, byte offset of the data section) of one shard file."""
        if shard not in self._hdrs:
            with open(os.path.join(self.base, shard), "rb") as f:
                n = int.from_bytes(f.read(8), "little")
                raw = f.read(n)
            if len(raw) != n:
                raise ValueError("%s: truncated safetensors header" % shard)
            h = json.loads(raw.decode("utf-8"))
            h.pop("__metadata__", None)
            self._hdrs[shard] = (h, 8 + n)
        return self._hdrs[shard]

    def __contains__(self, name):
        return name in self.index

    def names(self):
        return list(self.index)

    def info(self, name):
        if name not in self.index:
            raise KeyError("tensor %r not in %s" % (name, self.base))
        h, base = self.header(self.index[name])
        return h[name], base

    def _read(self, name, a, b):
        """Bytes [a, b) of a tensor's data."""
        info, base = self.info(name)
        with open(os.path.join(self.base, self.index[name]), "rb") as f:
            f.seek(base + info["data_offsets"][0] + a)
            raw = f.read(b - a)
        if len(raw) != b - a:
            raise ValueError("%s: tensor %r truncated" % (self.base, name))
        return raw

    @staticmethod
    def _decode(raw, dt, to_f16=False):
        if dt == "BF16":
            a = (np.frombuffer(raw, np.uint16).astype(np.uint32) << 16).view(np.float32)
        elif dt == "F16":
            a = np.frombuffer(raw, np.float16)
            return a.copy() if to_f16 else a.astype(np.float32)
        elif dt == "F32":
            a = np.frombuffer(raw, np.float32)
        elif dt == "I32":
            if to_f16:
                raise ValueError("an I32 tensor has no fp16 form")
            return np.frombuffer(raw, np.int32).copy()
        else:
            raise ValueError("safetensors dtype %s is not read by this loader" % dt)
        return a.astype(np.float16) if to_f16 else a.copy()

    def array(self, name, keep_f16=False):
        """The tensor as numpy: BF16/F16/F32 -> fp32 (F16 kept with `keep_f16`), I32 -> int32."""
        info, _ = self.info(name)
        a, z = info["data_offsets"]
        raw = self._read(name, 0, z - a)
        dt = info["dtype"]
        arr = self._decode(raw, dt, to_f16=keep_f16 and dt == "F16")
        return arr.reshape(info["shape"])

    def rows_f16(self, name, chunk_bytes=64 << 20):
        """A 2-D F16/BF16/F32 table as fp16 (rows, cols), read in row blocks of about
        `chunk_bytes` so no fp32 copy of the whole table exists."""
        info, _ = self.info(name)
        rows, cols = info["shape"]
        dt = info["dtype"]
        esz = {"F16": 2, "BF16": 2, "F32": 4}.get(dt)
        if esz is None:
            raise ValueError("%r: dtype %s is not a float table" % (name, dt))
        row = cols * esz
        rpc = max(1, chunk_bytes // row)
        out = np.empty((rows, cols), np.float16)
        for r0 in range(0, rows, rpc):
            r1 = min(rows, r0 + rpc)
            out[r0:r1] = self._decode(self._read(name, r0 * row, r1 * row), dt, to_f16=True).reshape(r1 - r0, cols)
        return out


def _text_config(cfg):
    """Composite configs nest the decoder under `text_config` (`webtorch/llm.py:428-432`)."""
    t = cfg.get("text_config") or {}
    return dict(t) if "hidden_size" in t else cfg


KV_BUDGET = 2 << 30  # bytes of fp32 K and V cache the automatic context length may take


def auto_lmax(requested, declared, L, NKV, HD):
    """Context length to load with (`webtorch/llm.py:1381-1395`): an explicit request, else what
    the model declares (2048 if nothing), capped by the KV-cache budget, at least 512."""
    if requested:
        return int(requested)
    per_tok = 2 * L * NKV * HD * 4
    cap = max(512, KV_BUDGET // per_tok)
    want = int(declared) if declared else 2048
    return max(512, min(want, cap))


def read_config(path):
    """config.json of a HuggingFace model directory, as a dict."""
    with open(os.path.join(str(path), "config.json")) as f:
        return json.load(f)


def is_quantized_dir(path):
    """Does the directory hold an already-quantized (AutoGPTQ) model (`quantization_config`),
    the test `from_pretrained` dispatches on (`webtorch/_sdk.py:108-113`)?"""
    full = read_config(path)
    return bool(full.get("quantization_config") or _text_config(full).get("quantization_config"))


def _shape_config(cfg, gs, bits):
    H, NH = int(cfg["hidden_size"]), int(cfg["num_attention_heads"])
    out = dict(L=int(cfg["num_hidden_layers"]), H=H, NH=NH, NKV=int(cfg.get("num_key_value_heads", NH)),
               HD=int(cfg.get("head_dim") or H // NH), I=int(cfg["intermediate_size"]),
               V=int(cfg["vocab_size"]), eps=float(cfg.get("rms_norm_eps", 1e-6)),
               theta=float(cfg.get("rope_theta", 10000.0)), gs=int(gs), bits=int(bits))
    ne = int(cfg.get("num_experts", cfg.get("num_local_experts", 0)) or 0)
    if ne:  # sparse MoE (`webtorch/llm.py:440-445, 477-479`)
        out.update(n_experts=ne, top_k=int(cfg.get("num_experts_per_tok", 0) or 0),
                   sparse_step=int(cfg.get("decoder_sparse_step", 1) or 1),
                   mlp_only=sorted(int(i) for i in (cfg.get("mlp_only_layers") or [])),
                   shared_expert=bool(cfg.get("shared_expert_intermediate_size", 0)))
    types = cfg.get("layer_types") or []
    if any(t != "full_attention" for t in types) or int(cfg.get("full_attention_interval", 0) or 0) > 1:
        raise NotImplementedError("hybrid linear-attention decoders are not part of this path")
    return out


def gptq_config(path):
    """Shape, quantization and context fields of an AutoGPTQ directory's config.json."""
    full = read_config(path)
    cfg = _text_config(full)
    q = full.get("quantization_config") or cfg.get("quantization_config")
    if not q:
        raise ValueError("%s: config.json has no quantization_config (not an AutoGPTQ directory)" % path)
    out = _shape_config(cfg, q["group_size"], q["bits"])
    return out, bool(cfg.get("tie_word_embeddings", False)), cfg.get("max_position_embeddings")


def _is_moe_layer(cfg, i):
    """`CausalLM._is_moe_layer` (`webtorch/llm.py:477-479`)."""
    return (cfg.get("n_experts", 0) > 0 and i not in cfg.get("mlp_only", [])
            and (i + 1) % cfg.get("sparse_step", 1) == 0)


def _decoder_layers(st, cfg, lin):
    """The layer dicts of `llm.CausalLM` read with the format's linear factory `lin(prefix)`, as
    `_build_layer` does (`webtorch/llm.py:506-539`): attention projections, optional per-head
    q/k RMSNorm weights (Qwen3), and either a dense SwiGLU or a sparse-MoE block (router
    `mlp.gate`, experts `mlp.experts.{e}.*`, optional shared expert and its gate)."""
    layers = []
    for i in range(cfg["L"]):
        p = "model.layers.%d." % i
        lay = {"q": lin(p + "self_attn.q_proj"), "k": lin(p + "self_attn.k_proj"),
               "v": lin(p + "self_attn.v_proj"), "o": lin(p + "self_attn.o_proj"),
               "in_ln": st.array(p + "input_layernorm.weight"),
               "post_ln": st.array(p + "post_attention_layernorm.weight")}
        for key, nm in (("qn", "self_attn.q_norm.weight"), ("kn", "self_attn.k_norm.weight")):
            if p + nm in st:
                lay[key] = st.array(p + nm)
        if _is_moe_layer(cfg, i):
            mo = {"router": lin(p + "mlp.gate"), "top_k": cfg["top_k"],
                  "experts": [{"gate": lin(p + "mlp.experts.%d.gate_proj" % e),
                               "up": lin(p + "mlp.experts.%d.up_proj" % e),
                               "down": lin(p + "mlp.experts.%d.down_proj" % e)} for e in range(cfg["n_experts"])]}
            if cfg.get("shared_expert"):
                mo["shared"] = {"gate": lin(p + "mlp.shared_expert.gate_proj"), "up": lin(p + "mlp.shared_expert.up_proj"),
                                "down": lin(p + "mlp.shared_expert.down_proj")}
                mo["shared_gate"] = _shared_gate(st, p + "mlp.shared_expert_gate", cfg)
            lay["moe"] = mo
        else:
            lay.update({"gate": lin(p + "mlp.gate_proj"), "up": lin(p + "mlp.up_proj"),
                        "down": lin(p + "mlp.down_proj")})
        layers.append(lay)
    return layers


def _shared_gate(st, prefix, cfg):
    """The shared expert's one-output gate: a linear of 1 column, quantized on load from its float
    weight with the output padded to the pack size (`QuantizedLinear.from_linear`)."""
    class _W:
        pass
    w = _W()
    w.weight = np.ascontiguousarray(st.array(prefix + ".weight").astype(np.float32).T)  # (in, out)
    w.bias = st.array(prefix + ".bias") if prefix + ".bias" in st else np.zeros(w.weight.shape[1], np.float32)
    return core.QuantizedLinear.from_linear(w, group_size=cfg["gs"], bits=cfg["bits"])


def gptq_weights(path):
    """`llm.CausalLM` weights from an AutoGPTQ safetensors directory, plus the model's
    declared context length: (weights, declared_lmax). A linear stored unquantized in such a
    directory (a MoE router kept in fp16, say) is quantized on load as `from_fp16` would."""
    cfg, tie, declared = gptq_config(path)
    st = SafetensorsDir(path)

    def lin(prefix):
        if prefix + ".qweight" not in st and prefix + ".weight" in st:
            return _quantize_linear(st, prefix, cfg["gs"], cfg["bits"])
        d = {"qweight": st.array(prefix + ".qweight"), "qzeros": st.array(prefix + ".qzeros"),
             "scales": st.array(prefix + ".scales", keep_f16=True)}
        if prefix + ".bias" in st:
            d["bias"] = st.array(prefix + ".bias")
        return d

    w = {"layers": _decoder_layers(st, cfg, lin), "embed": st.rows_f16("model.embed_tokens.weight"),
         "final_norm": st.array("model.norm.weight"), "cfg": cfg}
    if not tie:
        w["head"] = st.rows_f16("lm_head.weight")
    return w, declared


# ---------------------------------------------------------------------------------------------
# GGUF

GGUF_MAGIC = 0x46554747  # "GGUF", little-endian
# metadata value types
(GGUF_U8, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL, GGUF_STRING, GGUF_ARRAY,
 GGUF_U64, GGUF_I64, GGUF_F64) = range(13)
_SCALAR = {GGUF_U8: "<B", GGUF_I8: "<b", GGUF_U16: "<H", GGUF_I16: "<h", GGUF_U32: "<I", GGUF_I32: "<i",
           GGUF_F32: "<f", GGUF_U64: "<Q", GGUF_I64: "<q", GGUF_F64: "<d"}

# ggml tensor type ids and (values per block, bytes per block) of the types this package knows
GGML_TYPES = {0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20),
              6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 10: ("Q2_K", 256, 84),
              11: ("Q3_K", 256, 110), 12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176),
              14: ("Q6_K", 256, 210), 16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74),
              18: ("IQ3_XXS", 256, 98), 19: ("IQ1_S", 256, 50), 20: ("IQ4_NL", 32, 18),
              21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82), 23: ("IQ4_XS", 256, 136),
              29: ("IQ1_M", 256, 56), 30: ("BF16", 1, 2), 34: ("TQ1_0", 256, 54), 35: ("TQ2_0", 256, 66),
              39: ("MXFP4", 32, 17), 40: ("NVFP4", 64, 36), 41: ("Q1_0", 128, 18), 42: ("Q2_0", 64, 18)}
GGML_NAMES = {k: v[0] for k, v in GGML_TYPES.items()}
GGML_IDS = {v[0]: k for k, v in GGML_TYPES.items()}


def tensor_nbytes(ttype, n):
    """Bytes of n values of ggml type `ttype` (id or name); n must fill whole blocks."""
    tid = GGML_IDS[ttype] if isinstance(ttype, str) else int(ttype)
    if tid not in GGML_TYPES:
        raise NotImplementedError("ggml type %s" % ttype)
    _, vals, blk = GGML_TYPES[tid]
    if n % vals:
        raise ValueError("%d values do not fill whole %s blocks of %d" % (n, GGML_NAMES[tid], vals))
    return n // vals * blk


class _Cursor:
    """Little-endian reads over a byte buffer; EOFError past its end (the caller reads more)."""

    def __init__(self, buf):
        self.b = memoryview(buf)
        self.p = 0

    def take(self, n):
        if self.p + n > len(self.b):
            raise EOFError("GGUF header needs more than %d bytes" % len(self.b))
        v = self.b[self.p:self.p + n]
        self.p += n
        return v

    def scalar(self, fmt):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self):
        return bytes(self.take(self.scalar("<Q"))).decode("utf-8", "replace")

    def value(self, t):
        if t in _SCALAR:
            return self.scalar(_SCALAR[t])
        if t == GGUF_BOOL:
            return self.take(1)[0] != 0
        if t == GGUF_STRING:
            return self.string()
        if t == GGUF_ARRAY:
            at, n = self.scalar("<I"), self.scalar("<Q")
            return [self.value(at) for _ in range(n)]
        raise ValueError("bad GGUF metadata value type %d" % t)


def parse_header(buf):
    """(version, metadata, tensor_infos, data_start) of a GGUF file from a prefix `buf` of it
    (`webtorch/ggufload.py:92-112`). Tensor infos are dicts name / dims (ggml order, innermost
    first) / type / offset (from data_start). Raises EOFError when `buf` ends inside the
    header."""
    r = _Cursor(buf)
    if r.scalar("<I") != GGUF_MAGIC:
        raise ValueError("not a GGUF file")
    version = r.scalar("<I")
    if version < 2:
        raise NotImplementedError("GGUF version %d (64-bit counts need version >= 2)" % version)
    n_tensors, n_kv = r.scalar("<Q"), r.scalar("<Q")
    meta = {}
    for _ in range(n_kv):
        k = r.string()
        meta[k] = r.value(r.scalar("<I"))
    infos = []
    for _ in range(n_tensors):
        name = r.string()
        nd = r.scalar("<I")
        dims = [r.scalar("<Q") for _ in range(nd)]
        infos.append({"name": name, "dims": dims, "type": r.scalar("<I"), "offset": r.scalar("<Q")})
    align = int(meta.get("general.alignment", 32))
    return version, meta, infos, (r.p + align - 1) // align * align


class GGUFFile:
    """A GGUF file on disk: header parsed from a growing prefix, tensors read by byte range."""

    def __init__(self, path, first_read=1 << 20, max_header=128 << 20):
        self.path = str(path)
        size = first_read
        with open(self.path, "rb") as f:
            while True:
                f.seek(0)
                buf = f.read(size)
                try:
                    self.version, self.meta, infos, self.data_start = parse_header(buf)
                    break
                except EOFError:
                    if len(buf) < size or size >= max_header:
                        raise
                    size *= 2
        self.infos = {t["name"]: t for t in infos}

    def shape(self, name):
        """numpy order (outermost first), e.g. (out, in) for a 2-D weight."""
        return tuple(int(d) for d in reversed(self.infos[name]["dims"]))

    def type_name(self, name):
        t = self.infos[name]["type"]
        return GGML_NAMES.get(t, "type%d" % t)

    def raw(self, name):
        t = self.infos[name]
        n = int(np.prod([int(d) for d in t["dims"]], dtype=np.int64))
        nb = tensor_nbytes(t["type"], n)
        with open(self.path, "rb") as f:
            f.seek(self.data_start + int(t["offset"]))
            b = f.read(nb)
        if len(b) != nb:
            raise ValueError("%s: tensor %r truncated" % (self.path, name))
        return b

    def linear(self, name, bias=None):
        """The 2-D weight uploaded unchanged as a GGMLLinear (K = innermost dimension), or None
        when no native kernel decodes its type or K is not a whole number of blocks."""
        t = self.infos[name]
        if len(t["dims"]) != 2:
            return None
        nm = GGML_NAMES.get(t["type"])
        if not core.ggml_native_supported(nm):
            return None
        N, K = self.shape(name)
        if K % GGML_TYPES[t["type"]][1]:
            return None
        return core.GGMLLinear(self.raw(name), nm, K, N, bias)


def padded_dims(K, N, gs, bits):
    """(Kp, Np): K padded to the group multiple (group times pack factor when the group is not a
    multiple of it) and N to the pack factor, as `_gquant` / `_gload_quant` pad
    (`webtorch/llm.py:805-828, 843-849`)."""
    per = 32 // bits
    kmul = gs if gs % per == 0 else gs * per
    return K + (-K) % kmul, N + (-N) % per


def _quantize_out_in(W, gs, bits, bias=None):
    """(N, K) float device weight -> GPTQ layer dict quantized on the device (`_gquant`,
    `webtorch/llm.py:835-853`: zero offset 0, fp32 scales), zero-padded to (Np, Kp) first. The
    padded rows quantize to codes equal to their zero point (value 0 exactly) and the padded
    columns are dropped by the layer; the dict carries the true K and N as "Kt" / "Nt"."""
    import torch
    N, K = int(W.shape[0]), int(W.shape[1])
    Kp, Np = padded_dims(K, N, gs, bits)
    if (Kp, Np) != (K, N):
        W = torch.nn.functional.pad(W, (0, Kp - K, 0, Np - N))
    qw, qz, sc, _, _ = core.gptq_quantize(W.contiguous(), gs, bits, from_out_in=True)
    return {"qweight": qw, "qzeros": qz, "scales": sc, "zoff": 0.0, "bias": bias, "Kt": K, "Nt": N}


def _quantize_linear(st, prefix, gs, bits):
    """One float (out, in) linear of a safetensors directory quantized on the device in its file
    encoding (`_gquant`, `webtorch/llm.py:835-853`: gs 128, zero offset 0, fp32 scales, K and N
    padded to the group / pack size)."""
    import torch
    W = torch.from_numpy(st.array(prefix + ".weight", keep_f16=True)).to(core.device())
    b = st.array(prefix + ".bias") if prefix + ".bias" in st else None
    return _quantize_out_in(W, gs, bits, b)


def fp16_weights(path, bits, gs=128):
    """`llm.CausalLM` weights of a plain fp16/bf16 HuggingFace directory quantized on load to
    int`bits` (`from_fp16(quantize=bits)`, `webtorch/llm.py:1211-1257`): every (out, in)
    projection goes to the device in its file encoding and is quantized there by
    `core.gptq_quantize` -- the reference's `_gquant` (`webtorch/llm.py:835-853`): group size
    128, asymmetric min-max, zero offset 0, fp32 scales; int8 is the same rule with 8-bit codes.
    Returns (weights, declared context length)."""
    full = read_config(path)
    cfg = _text_config(full)
    if full.get("quantization_config") or cfg.get("quantization_config"):
        raise ValueError("%s holds an already-quantized model; load it with from_gptq" % path)
    if int(bits) not in (4, 8):
        raise NotImplementedError("quantize-on-load to %s bits (4 or 8)" % bits)
    shape = _shape_config(cfg, gs, bits)
    st = SafetensorsDir(path)
    w = {"layers": _decoder_layers(st, shape, lambda prefix: _quantize_linear(st, prefix, gs, int(bits))),
         "embed": st.rows_f16("model.embed_tokens.weight"), "final_norm": st.array("model.norm.weight"),
         "cfg": shape}
    if not cfg.get("tie_word_embeddings", False):
        w["head"] = st.rows_f16("lm_head.weight")
    return w, cfg.get("max_position_embeddings")


# ---- GGUF models -----------------------------------------------------------------------------

def gguf_source_bits(g):
    """The integer width that keeps what a GGUF stores (`_source_bits`, `webtorch/llm.py:296-320`):
    8 when the block type holding the most layer weights (counted by element) takes more than 4.5
    bits per weight, else 4."""
    weight = {}
    for name, t in g.infos.items():
        if name.startswith("blk."):
            weight[t["type"]] = weight.get(t["type"], 0) + int(np.prod([int(d) for d in t["dims"]], dtype=np.int64))
    if not weight:
        return 4
    dom = max(weight, key=weight.get)
    return 8 if tensor_nbytes(dom, 4096) * 8.0 / 4096 > 4.5 else 4


def gguf_dequant(raw, ttype, n):
    """fp32 device tensor of the first n values of a GGUF byte stream of type `ttype` (id):
    block types through the device decoders (bit-exact with `ggufload.dequant`), F32 / F16 / BF16
    by conversion."""
    import torch
    name = GGML_NAMES.get(int(ttype), "type%d" % int(ttype))
    b = np.frombuffer(raw, np.uint8) if isinstance(raw, (bytes, bytearray, memoryview)) else np.asarray(raw, np.uint8)
    if name == "F32":
        return torch.from_numpy(b[:4 * n].view(np.float32).copy()).to(core.device())
    if name == "F16":
        return torch.from_numpy(b[:2 * n].view(np.float16).copy()).to(core.device()).float()
    if name == "BF16":
        u = b[:2 * n].view(np.uint16).astype(np.uint32) << 16
        return torch.from_numpy(u.view(np.float32)).to(core.device())
    nb = tensor_nbytes(int(ttype), n)
    blocks = torch.from_numpy(b[:nb].copy()).to(core.device())
    vals = GGML_TYPES[int(ttype)][1]
    if name == "Q4_K":
        return core.q4k_dequant(blocks, n // vals)
    if not core.ggml_native_supported(name):
        raise NotImplementedError("GGUF type %s has no decoder here" % name)
    return core.ggml_dequant(blocks, name, n // vals)


def _gguf_requant(W, bits, gs, bias):
    """fp32 (out, in) device weight -> GPTQ layer dict quantized on the device (`_gload_quant`,
    `webtorch/llm.py:787-833`: zero offset 0, fp32 scales, padded to the group / pack size)."""
    return _quantize_out_in(W, gs, bits, bias)


def _gguf_linear(g, name, bits, gs, weights, bias=None):
    """One 2-D GGUF weight as a layer: uploaded unchanged for a native kernel (`_gload_native`,
    `webtorch/llm.py:763-785`) when `weights` is "native" and its type has one, else decoded on the
    device and quantized to int`bits` (`_gload_quant`, `webtorch/llm.py:787-833`)."""
    if weights == "native":
        lin = g.linear(name, bias)
        if lin is not None:
            return lin
    t = g.infos[name]
    shape = g.shape(name)
    if len(shape) != 2:
        raise NotImplementedError("%s is %d-D, a linear weight is 2-D" % (name, len(shape)))
    W = gguf_dequant(g.raw(name), t["type"], shape[0] * shape[1]).reshape(shape)
    return _gguf_requant(W, bits, gs, bias)


def _gguf_experts(g, name, bits, gs, weights):
    """The experts of a stacked `ffn_*_exps` tensor (ggml dims in, out, E), one at a time: each
    expert's bytes are a block-aligned slice (`_gexperts`, `webtorch/llm.py:731-760`). With
    `weights="native"` a slice whose block type has a kernel here (and whose K is a whole number
    of blocks) stays in its encoding as a GGMLLinear, as the reference uploads it; otherwise it is
    decoded on the device and quantized to int`bits` for the GPTQ expert kernels."""
    t = g.infos[name]
    E, N, K = g.shape(name)
    per = N * K
    nb = tensor_nbytes(t["type"], per)
    raw = g.raw(name)
    nm = GGML_NAMES.get(t["type"])
    if weights == "native" and core.ggml_native_supported(nm) and nm not in core.DENSE_TYPES \
            and K % GGML_TYPES[t["type"]][1] == 0:
        return [core.GGMLLinear(raw[e * nb:(e + 1) * nb], nm, K, N) for e in range(E)]
    return [_gguf_requant(gguf_dequant(raw[e * nb:(e + 1) * nb], t["type"], per).reshape(N, K), bits, gs, None)
            for e in range(E)]


def gguf_weights(path, bits=None, weights="native", gs=128):
    """Engine weights of a llama.cpp GGUF decoder (`CausalLM.from_gguf`, `webtorch/llm.py:
    856-1129`): shape, RoPE and norm settings from the file's `{arch}.*` metadata, QK-norm and
    sparse-MoE blocks detected from the tensors. Returns (weights, declared context length).

    `bits=None` takes the width from the file (`gguf_source_bits`). `weights="native"` keeps every
    2-D weight whose block type has a kernel here in its file encoding (GGMLLinear) and quantizes
    the rest to int`bits`; "requant" quantizes all of them. The embedding is decoded once to an
    exact fp32 table on the device; the head is the file's `output.weight` or, when absent, the
    embedding (tied), native or quantized like the other weights. Experts follow the same rule
    (`_gexperts`): native slices run the grouped GGUF expert GEMV; should one projection of a
    layer be native and another not (a K that is not a whole number of blocks), the layer's
    experts are all quantized, since one layer runs one expert kernel. Recurrent / state-space
    blocks and partial RoPE are not part of this engine and raise NotImplementedError."""
    if weights not in ("native", "requant"):
        raise ValueError("weights must be 'native' or 'requant', got %r" % (weights,))
    g = GGUFFile(path)
    arch = g.meta.get("general.architecture")
    if not arch:
        raise ValueError("GGUF has no general.architecture")
    A = arch + "."

    def m(key, default=None, required=True):
        if A + key in g.meta:
            return g.meta[A + key]
        if default is not None or not required:
            return default
        raise NotImplementedError("GGUF arch %r is missing %r" % (arch, key))

    bad = sorted({GGML_NAMES.get(t["type"], "type%d" % t["type"]) for t in g.infos.values()
                  if t["type"] not in GGML_TYPES})
    if bad:
        raise NotImplementedError("GGUF uses quantization type(s) %s this package cannot decode" % ", ".join(bad))
    H = int(m("embedding_length"))
    L = int(m("block_count")) - int(m("nextn_predict_layers", 0) or 0)
    NH = int(m("attention.head_count"))
    NKV = int(m("attention.head_count_kv", NH) or NH)
    HD = int(m("attention.key_length", 0, required=False) or H // NH)
    if int(m("rope.dimension_count", 0, required=False) or HD) != HD:
        raise NotImplementedError("partial RoPE (rope.dimension_count < head dim) is not part of this engine")
    if m("full_attention_interval", 0, required=False) or m("attention.recurrent_layers", None, required=False) \
            or any(n.startswith("blk.0.ssm_") for n in g.infos):
        raise NotImplementedError("recurrent / state-space blocks are not part of this engine")
    bits = int(bits) if bits else gguf_source_bits(g)
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    f32 = lambda n: gguf_dequant(g.raw(n), g.infos[n]["type"], int(np.prod(g.shape(n))))  # noqa: E731
    opt = lambda n: f32(n) if n in g.infos else None  # noqa: E731
    lin = lambda n, b=None: _gguf_linear(g, n, bits, gs, weights, b)  # noqa: E731
    top_k = int(m("expert_used_count", 0, required=False) or 0)
    layers, I = [], int(m("feed_forward_length", 0, required=False) or 0)
    moe_I = int(m("expert_feed_forward_length", 0, required=False) or 0)
    for i in range(L):
        p = "blk.%d." % i
        post = next((n for n in ("ffn_norm", "post_attention_norm") if p + n + ".weight" in g.infos), None)
        if post is None or p + "attn_norm.weight" not in g.infos:
            raise NotImplementedError("GGUF block %d lacks attn_norm / ffn_norm" % i)
        if not all(p + "attn_%s.weight" % x in g.infos for x in ("q", "k", "v")):
            raise NotImplementedError("GGUF block %d has no separate attn_q / attn_k / attn_v" % i)
        lay = {"in_ln": f32(p + "attn_norm.weight"), "post_ln": f32(p + post + ".weight"),
               "qn": opt(p + "attn_q_norm.weight"), "kn": opt(p + "attn_k_norm.weight")}
        for key, nm in (("q", "attn_q"), ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output")):
            lay[key] = lin(p + nm + ".weight", opt(p + nm + ".bias"))
        if p + "ffn_gate_inp.weight" in g.infos:  # sparse MoE: router + stacked experts
            ex = {k: _gguf_experts(g, p + "ffn_%s_exps.weight" % k, bits, gs, weights) for k in ("gate", "up", "down")}
            if len({isinstance(ex[k][0], core.GGMLLinear) for k in ex}) != 1:  # one expert kernel per layer
                ex = {k: _gguf_experts(g, p + "ffn_%s_exps.weight" % k, bits, gs, "requant") for k in ex}
            E = len(ex["gate"])
            moe_I = moe_I or g.shape(p + "ffn_gate_exps.weight")[1]
            lay["moe"] = {"router": lin(p + "ffn_gate_inp.weight"), "top_k": top_k or 2,
                          "experts": [{k: ex[k][e] for k in ex} for e in range(E)]}
        else:
            for key, nm in (("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down")):
                lay[key] = lin(p + nm + ".weight")
            I = I or g.shape(p + "ffn_gate.weight")[0]
        layers.append(lay)
    V, He = g.shape("token_embd.weight")
    if He != H:
        raise ValueError("token_embd is (%d, %d), embedding_length %d" % (V, He, H))
    embed = f32("token_embd.weight").reshape(V, H)
    head = lin("output.weight" if "output.weight" in g.infos else "token_embd.weight")
    cfg = dict(L=L, H=H, NH=NH, NKV=NKV, HD=HD, I=I or moe_I, V=V, gs=gs, bits=bits,
               eps=float(m("attention.layer_norm_rms_epsilon", 1e-6, required=False)),
               theta=float(m("rope.freq_base", 10000.0, required=False)))
    if moe_I:
        cfg.update(n_experts=len(layers[-1]["moe"]["experts"]) if "moe" in layers[-1] else 0, moe_I=moe_I, top_k=top_k)
    return ({"layers": layers, "embed": embed, "head_linear": head, "final_norm": f32("output_norm.weight"),
             "cfg": cfg}, m("context_length", None, required=False))
