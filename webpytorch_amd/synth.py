"""Seeded synthetic weights and activations for the quantized-linear workloads.

Every tensor comes from its own `numpy.random.default_rng((seed, tag))` stream, so a given
(seed, shape) always yields the same bytes on any host. Nothing here touches the GPU; the
results are plain numpy arrays in the on-disk layouts the loaders accept:

* GPTQ (AutoGPTQ) -- qweight int32 (K/per, N) holding `per = 32/bits` rows of a column per
  word, row k at bit offset (k % per) * bits (`webtorch/quantize.py:96-106`); qzeros int32
  (K/gs, N/per) packed along N; scales fp16 (K/gs, N); g_idx int32 (K,).
* GGUF Q4_K -- 144-byte super-blocks of 256 weights: fp16 d, fp16 dmin, 12 bytes of packed
  6-bit sub-block scales/mins (the layout `get_scale_min_k4` reads,
  `webtorch/ggufload.py:120-130`), then 128 bytes of 4-bit quants.
"""
import zlib

import numpy as np

# Distinct stream tags so that two tensors of one workload never share random bits.
_TAGS = {}


def rng(seed, tag):
    """Independent generator for tensor `tag` of workload `seed`."""
    t = _TAGS.get(tag)
    if t is None:
        t = _TAGS[tag] = zlib.crc32(tag.encode()) & 0x7FFFFFFF
    return np.random.default_rng((int(seed), t))


def random_words(g, shape):
    """int32 array of uniformly random bits (so every packed nibble/byte is uniform)."""
    return g.integers(0, 1 << 32, size=shape, dtype=np.uint64).astype(np.uint32).view(np.int32)


def gptq_scales(g, shape):
    """fp16 scales = |N(0,1)| * 0.01 + 1e-3."""
    return (np.abs(g.standard_normal(shape)) * 0.01 + 1e-3).astype(np.float16)


def gptq_layer(seed, K, N, gs=128, bits=4, act_order=False, name="w"):
    """Random AutoGPTQ layer: uniform packed codes, uniform stored zeros, |N|*0.01+1e-3 scales.

    With `act_order`, g_idx is a seeded permutation of arange(K)//gs (desc_act=True)."""
    per = 32 // bits
    if K % per or N % per or K % gs:
        raise ValueError("K must divide by group size and pack factor, N by pack factor")
    qweight = random_words(rng(seed, name + ".qweight"), (K // per, N))
    qzeros = random_words(rng(seed, name + ".qzeros"), (K // gs, N // per))
    scales = gptq_scales(rng(seed, name + ".scales"), (K // gs, N))
    g_idx = (np.arange(K, dtype=np.int32) // gs).astype(np.int32)
    if act_order:
        g_idx = rng(seed, name + ".g_idx").permutation(g_idx).astype(np.int32)
    return {"qweight": qweight, "qzeros": qzeros, "scales": scales, "g_idx": g_idx,
            "K": K, "N": N, "gs": gs, "bits": bits}


def int8_per_channel_layer(seed, K, N, name="w8"):
    """Per-output-channel symmetric int8 (q ~ U[-127,127], fp16 scales |N|*0.01), written in
    the GPTQ int8 layout with one group spanning all of K: stored code u = q + 128, stored
    zero 127 (zero_offset 1 makes the effective zero 128), so s * (u - 128) = s * q."""
    g = rng(seed, name + ".q")
    q = g.integers(-127, 128, size=(K, N), dtype=np.int32)
    u = (q + 128).astype(np.uint32)
    qweight = np.zeros((K // 4, N), np.uint32)
    for r in range(4):
        qweight |= u[r::4] << np.uint32(8 * r)
    qzeros = np.full((1, N // 4), 0x7F7F7F7F, np.uint32)
    scales = (np.abs(rng(seed, name + ".scales").standard_normal((1, N))) * 0.01).astype(np.float16)
    return {"qweight": qweight.view(np.int32), "qzeros": qzeros.view(np.int32), "scales": scales,
            "g_idx": np.zeros(K, np.int32), "K": K, "N": N, "gs": K, "bits": 8, "q": q}


def pack_q4k_scales(sc, m):
    """Inverse of `get_scale_min_k4`: 8 six-bit scales and 8 six-bit mins -> 12 bytes/block.

    sc, m: (blocks, 8) integer arrays in 0..63. Bytes 0-3 hold sc[0..3] plus the top two bits
    of sc[4..7]; bytes 4-7 hold m[0..3] plus the top two bits of m[4..7]; bytes 8-11 hold the
    low nibbles of sc[4..7] (low half) and m[4..7] (high half)."""
    sc = np.asarray(sc, np.uint8); m = np.asarray(m, np.uint8)
    out = np.empty((sc.shape[0], 12), np.uint8)
    out[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 15) | ((m[:, 4:8] & 15) << 4)
    return out


def q4k_blocks(seed, n_blocks, name="q4k"):
    """Random Q4_K super-blocks as a (n_blocks, 144) uint8 array.

    d, dmin = fp16 |N(0,1)|*0.01; sub-block scales and mins uniform over 0..63; quants
    uniform random bytes."""
    d = (np.abs(rng(seed, name + ".d").standard_normal(n_blocks)) * 0.01).astype(np.float16)
    dmin = (np.abs(rng(seed, name + ".dmin").standard_normal(n_blocks)) * 0.01).astype(np.float16)
    g = rng(seed, name + ".sm")
    sc = g.integers(0, 64, size=(n_blocks, 8), dtype=np.uint8)
    m = g.integers(0, 64, size=(n_blocks, 8), dtype=np.uint8)
    qs = rng(seed, name + ".qs").integers(0, 256, size=(n_blocks, 128), dtype=np.uint8)
    blk = np.empty((n_blocks, 144), np.uint8)
    blk[:, 0:2] = d.view(np.uint8).reshape(n_blocks, 2)
    blk[:, 2:4] = dmin.view(np.uint8).reshape(n_blocks, 2)
    blk[:, 4:16] = pack_q4k_scales(sc, m)
    blk[:, 16:144] = qs
    return blk


def q4k_layer(seed, K, N, name="q4k"):
    """Q4_K weight of N rows by K columns: row n is K/256 consecutive super-blocks."""
    if K % 256:
        raise ValueError("Q4_K needs K % 256 == 0")
    return q4k_blocks(seed, N * (K // 256), name).reshape(N, (K // 256) * 144)


def q8_0_layer(seed, K, N, name="q8_0"):
    """N rows of K/32 GGUF Q8_0 blocks (34 bytes: fp16 d = |N(0,1)| * 0.01, 32 uniform int8
    codes), as a (N, K/32 * 34) uint8 array."""
    g = rng(seed, name)
    nb = N * (K // 32)
    b = np.empty((nb, 34), np.uint8)
    b[:, 0:2] = (np.abs(g.standard_normal(nb)) * 0.01).astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[:, 2:] = g.integers(0, 256, (nb, 32), dtype=np.uint8)
    return b.reshape(N, (K // 32) * 34)


def q6k_layer(seed, K, N, name="q6k"):
    """N rows of K/256 GGUF Q6_K super-blocks (210 bytes: uniform ql and qh bytes, 16 int8
    scales uniform in [-64, 63], fp16 d = |N(0,1)| * 0.001), as a (N, K/256 * 210) uint8 array."""
    g = rng(seed, name)
    nb = N * (K // 256)
    b = np.empty((nb, 210), np.uint8)
    b[:, 0:192] = g.integers(0, 256, (nb, 192), dtype=np.uint8)
    b[:, 192:208] = g.integers(-64, 64, (nb, 16)).astype(np.int8).view(np.uint8)
    b[:, 208:210] = (np.abs(g.standard_normal(nb)) * 0.001).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(N, (K // 256) * 210)


# (values, bytes, byte offsets of the fp16 scale fields) of the GGUF block types
GGML_BLOCKS = {"Q4_0": (32, 18, (0,)), "Q4_1": (32, 20, (0, 2)), "Q5_0": (32, 22, (0,)),
               "Q5_1": (32, 24, (0, 2)), "Q8_0": (32, 34, (0,)), "IQ4_NL": (32, 18, (0,)),
               "IQ4_XS": (256, 136, (0,)), "Q2_K": (256, 84, (80, 82)), "Q3_K": (256, 110, (108,)),
               "Q4_K": (256, 144, (0, 2)), "Q5_K": (256, 176, (0, 2)), "Q6_K": (256, 210, (208,)),
               "IQ2_XXS": (256, 66, (0,)), "IQ2_XS": (256, 74, (0,)), "IQ2_S": (256, 82, (0,)),
               "IQ3_XXS": (256, 98, (0,)), "IQ3_S": (256, 110, (0,)), "IQ1_S": (256, 50, (0,)),
               "IQ1_M": (256, 56, ()), "TQ1_0": (256, 54, (52,)), "TQ2_0": (256, 66, (64,)),
               "MXFP4": (32, 17, ()), "NVFP4": (64, 36, ()), "Q1_0": (128, 18, (0,)), "Q2_0": (64, 18, (0,))}
# unquantized matrices: bytes per value
DENSE_TYPES = {"F32": 4, "F16": 2, "BF16": 2}


def _scale_fields(type_name, b, g, scale):
    """Scale fields that are not a plain fp16: MXFP4's E8M0 exponent byte, NVFP4's four UE4M3
    bytes and IQ1_M's fp16 d spread over the top nibbles of its scale words, drawn so the values
    stay finite and near `scale`."""
    nb = b.shape[0]
    if type_name == "MXFP4":  # value = code * 2^(e - 128), codes up to 12
        e0 = int(round(128 + np.log2(scale / 4)))
        b[:, 0] = np.clip(e0 + g.integers(-2, 3, nb), 1, 254).astype(np.uint8)
    elif type_name == "NVFP4":  # value = code * (8 + m) 2^(e - 11), e > 0
        e0 = int(round(11 + np.log2(scale / 48)))
        e = np.clip(e0 + g.integers(-1, 2, (nb, 4)), 0, 14)
        b[:, 0:4] = ((e << 3) | g.integers(0, 8, (nb, 4))).astype(np.uint8)
    elif type_name == "IQ1_M":  # d's fp16 bits: nibble k in the top of scale word k
        d = (np.abs(g.standard_normal(nb)) * scale).astype(np.float16).view(np.uint16).astype(np.int64)
        for k in range(4):
            hi = 49 + 2 * k
            b[:, hi] = ((b[:, hi] & 0x0F) | (((d >> (4 * k)) & 15) << 4)).astype(np.uint8)


def ggml_layer(type_name, seed, K, N, scale=0.002):
    """N rows of K / block-values blocks of a GGUF type: uniform code and sub-scale bytes, every
    fp16 scale field |N(0,1)| * scale (finite, so the weight is too), as a uint8 (N, row bytes)
    array."""
    g = rng(seed, "ggml-" + type_name)
    if type_name in DENSE_TYPES:  # values ~ N(0, (4 scale)^2) in the stored encoding
        w = (g.standard_normal((N, K)) * 4 * scale).astype(np.float32)
        if type_name == "F16":
            w = w.astype(np.float16)
        elif type_name == "BF16":
            w = (w.view(np.uint32) >> 16).astype(np.uint16)
        return np.ascontiguousarray(w).view(np.uint8).reshape(N, K * DENSE_TYPES[type_name])
    vals, nbytes, f16 = GGML_BLOCKS[type_name]
    if K % vals:
        raise ValueError("%s needs K %% %d == 0" % (type_name, vals))
    nb = N * (K // vals)
    b = g.integers(0, 256, (nb, nbytes), dtype=np.uint8)
    for off in f16:
        b[:, off:off + 2] = (np.abs(g.standard_normal(nb)) * scale).astype(np.float16).view(np.uint8).reshape(nb, 2)
    _scale_fields(type_name, b, g, scale)
    return b.reshape(N, (K // vals) * nbytes)


def activations(seed, M, K, dtype=np.float16, name="x"):
    return rng(seed, name).standard_normal((M, K)).astype(dtype)


# ---- workload shapes ------------------------------------------------------------------
QWEN2_05B = dict(L=24, H=896, NH=14, NKV=2, HD=64, I=4864, V=151936, eps=1e-6,
                 theta=1e6, gs=128, bits=4)


def moe_workload(seed, T=256, H=2048, E=128, I=768, top_k=8, gs=128, experts=True):
    """Qwen3-MoE-shaped expert block: tokens, router logits and E int4 experts."""
    x = activations(seed, T, H, np.float16, "moe.x")
    logits = rng(seed, "moe.logits").standard_normal((T, E)).astype(np.float32)
    ex = None
    if experts:
        ex = [{"gate": gptq_layer(seed, H, I, gs, 4, name="moe.%d.gate" % e),
               "up": gptq_layer(seed, H, I, gs, 4, name="moe.%d.up" % e),
               "down": gptq_layer(seed, I, H, gs, 4, name="moe.%d.down" % e)}
              for e in range(E)]
    return {"x": x, "logits": logits, "experts": ex, "top_k": top_k, "T": T, "H": H,
            "E": E, "I": I, "gs": gs}


def quantized_gaussian_layer(seed, K, N, gs=128, bits=4, name="w"):
    """AutoGPTQ layer quantized from Gaussian weights ~N(0, 1/K) with the asymmetric min-max
    rule (per group and column: scale = (max - min) / qmax, zero = round(-min / scale)), stored
    as AutoGPTQ does (zero - 1, fp16 scales). Unlike uniform random codes, these weights have
    no common offset, so a model built from them produces varied greedy tokens."""
    per, qmax = 32 // bits, (1 << bits) - 1
    W = rng(seed, name + ".w").standard_normal((K, N)) / np.sqrt(K)
    Wg = W.reshape(K // gs, gs, N)
    lo, hi = Wg.min(1), Wg.max(1)
    sc = ((hi - lo) / qmax).astype(np.float16)
    s32 = sc.astype(np.float64)
    zp = np.clip(np.round(-lo / s32), 1, qmax).astype(np.int64)   # AutoGPTQ cannot store zero 0
    q = np.clip(np.round(Wg / s32[:, None, :]) + zp[:, None, :], 0, qmax).astype(np.int64).reshape(K, N)
    qweight = np.zeros((K // per, N), np.uint32)
    for j in range(per):
        qweight |= q[j::per].astype(np.uint32) << np.uint32(j * bits)
    zs = ((zp - 1) & qmax).astype(np.uint32)
    qzeros = np.zeros((K // gs, N // per), np.uint32)
    for j in range(per):
        qzeros |= zs[:, j::per] << np.uint32(j * bits)
    return {"qweight": qweight.view(np.int32), "qzeros": qzeros.view(np.int32), "scales": sc,
            "g_idx": (np.arange(K) // gs).astype(np.int32), "K": K, "N": N, "gs": gs, "bits": bits}


def decoder_weights(seed, L=24, H=896, NH=14, NKV=2, HD=64, I=4864, V=151936, gs=128,
                    bits=4, embed_scale=0.02, gaussian=False, n_experts=0, moe_I=None, top_k=2,
                    qk_norm=False, **_):
    """Random-init Qwen2-shaped int4 decoder: AutoGPTQ int4 linears (q/k/v with fp16 bias),
    RMSNorm weights near 1, fp16 embeddings ~N(0, embed_scale**2) (the head is tied to them).
    The linears hold uniform random codes, zeros and |N|*0.01+1e-3 scales, or, with
    `gaussian`, codes quantized from Gaussian weights (`quantized_gaussian_layer`).

    `n_experts` > 0 makes every layer's MLP a sparse MoE block (Qwen3-MoE style): a router
    linear H -> n_experts and n_experts {gate, up, down} experts of intermediate `moe_I`, top
    `top_k`, stored under "moe". `qk_norm` adds the per-head q/k RMSNorm weights "qn"/"kn"
    (fp16 [HD], near 1)."""
    make = (lambda K, N, name: quantized_gaussian_layer(seed, K, N, gs, bits, name=name)) if gaussian else \
        (lambda K, N, name: gptq_layer(seed, K, N, gs, bits, name=name))
    layers = []
    for i in range(L):
        p = "l%d." % i
        lay = {"q": make(H, NH * HD, p + "q"), "k": make(H, NKV * HD, p + "k"),
               "v": make(H, NKV * HD, p + "v"), "o": make(NH * HD, H, p + "o")}
        if n_experts:
            mi = moe_I or I
            lay["moe"] = {"router": make(H, n_experts, p + "router"), "top_k": int(top_k),
                          "experts": [{"gate": make(H, mi, p + "e%d.gate" % e), "up": make(H, mi, p + "e%d.up" % e),
                                       "down": make(mi, H, p + "e%d.down" % e)} for e in range(n_experts)]}
        else:
            lay.update({"gate": make(H, I, p + "gate"), "up": make(H, I, p + "up"), "down": make(I, H, p + "down")})
        if qk_norm:
            lay["qn"] = (1.0 + 0.1 * rng(seed, p + "qn").standard_normal(HD)).astype(np.float16)
            lay["kn"] = (1.0 + 0.1 * rng(seed, p + "kn").standard_normal(HD)).astype(np.float16)
        for nm, n in (("q", NH * HD), ("k", NKV * HD), ("v", NKV * HD)):
            lay[nm]["bias"] = (rng(seed, p + nm + ".bias").standard_normal(n) * 0.02).astype(np.float16)
        lay["in_ln"] = (1.0 + 0.02 * rng(seed, p + "in_ln").standard_normal(H)).astype(np.float16)
        lay["post_ln"] = (1.0 + 0.02 * rng(seed, p + "post_ln").standard_normal(H)).astype(np.float16)
        layers.append(lay)
    embed = (rng(seed, "embed").standard_normal((V, H)) * embed_scale).astype(np.float16)
    final_norm = (1.0 + 0.02 * rng(seed, "final_norm").standard_normal(H)).astype(np.float16)
    cfg = dict(L=L, H=H, NH=NH, NKV=NKV, HD=HD, I=I, V=V, gs=gs, bits=bits)
    if n_experts:
        cfg.update(n_experts=int(n_experts), moe_I=int(moe_I or I), top_k=int(top_k))
    return {"layers": layers, "embed": embed, "final_norm": final_norm, "cfg": cfg}


def prompt_ids(seed, T=64, V=151936):
    return rng(seed, "prompt").integers(0, V, size=T).astype(np.int64)


def fp16_decoder(seed, L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, eps=1e-6, theta=1e6, max_pos=4096,
                 n_experts=0, moe_I=0, top_k=0, mlp_only=(), **_):
    """A plain (unquantized) fp16 Qwen2-shaped model as a HuggingFace directory holds it: the
    tensors by their HF names, (out, in) projection weights ~N(0, 1/in), q/k/v biases, RMSNorm
    weights near 1, embeddings ~N(0, 0.02**2) with the head tied to them, and the config.json
    fields. With `n_experts`, the layers not in `mlp_only` are Qwen-MoE sparse blocks: a router
    `mlp.gate` (E, H) ~N(0, 1/H) and experts `mlp.experts.{e}.{gate,up,down}_proj` of
    intermediate `moe_I`. Returns {"tensors": {name: fp16 array}, "config": dict}."""
    t = {"model.embed_tokens.weight": (rng(seed, "embed").standard_normal((V, H)) * 0.02).astype(np.float16),
         "model.norm.weight": (1.0 + 0.02 * rng(seed, "final_norm").standard_normal(H)).astype(np.float16)}
    projs = (("self_attn.q_proj", NH * HD, H, True), ("self_attn.k_proj", NKV * HD, H, True),
             ("self_attn.v_proj", NKV * HD, H, True), ("self_attn.o_proj", H, NH * HD, False),
             ("mlp.gate_proj", I, H, False), ("mlp.up_proj", I, H, False), ("mlp.down_proj", H, I, False))
    for i in range(L):
        p = "model.layers.%d." % i
        sparse = n_experts and i not in mlp_only
        for nm, n_out, n_in, bias in projs:
            if sparse and nm.startswith("mlp."):
                continue
            t[p + nm + ".weight"] = (rng(seed, p + nm).standard_normal((n_out, n_in)) / np.sqrt(n_in)).astype(np.float16)
            if bias:
                t[p + nm + ".bias"] = (rng(seed, p + nm + ".bias").standard_normal(n_out) * 0.02).astype(np.float16)
        if sparse:
            t[p + "mlp.gate.weight"] = (rng(seed, p + "router").standard_normal((n_experts, H)) / np.sqrt(H)).astype(
                np.float16)
            for e in range(n_experts):
                for nm, n_out, n_in in (("gate_proj", moe_I, H), ("up_proj", moe_I, H), ("down_proj", H, moe_I)):
                    q = p + "mlp.experts.%d.%s" % (e, nm)
                    t[q + ".weight"] = (rng(seed, q).standard_normal((n_out, n_in)) / np.sqrt(n_in)).astype(np.float16)
        t[p + "input_layernorm.weight"] = (1.0 + 0.02 * rng(seed, p + "in_ln").standard_normal(H)).astype(np.float16)
        t[p + "post_attention_layernorm.weight"] = (
            1.0 + 0.02 * rng(seed, p + "post_ln").standard_normal(H)).astype(np.float16)
    cfg = {"architectures": ["Qwen2ForCausalLM"], "model_type": "qwen2", "hidden_size": H,
           "intermediate_size": I, "num_hidden_layers": L, "num_attention_heads": NH,
           "num_key_value_heads": NKV, "head_dim": HD, "vocab_size": V, "rms_norm_eps": eps,
           "rope_theta": theta, "tie_word_embeddings": True, "max_position_embeddings": max_pos,
           "torch_dtype": "float16"}
    if n_experts:
        cfg.update({"architectures": ["Qwen2MoeForCausalLM"], "model_type": "qwen2_moe", "num_experts": n_experts,
                    "num_experts_per_tok": top_k, "moe_intermediate_size": moe_I, "norm_topk_prob": True,
                    "decoder_sparse_step": 1, "mlp_only_layers": sorted(mlp_only)})
    return {"tensors": t, "config": cfg}
