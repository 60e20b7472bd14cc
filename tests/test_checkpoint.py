"""On-disk checkpoints: the safetensors reader against files written by the `safetensors`
package (an independent implementation of the format) and by hand from the format's spec
(BF16), the AutoGPTQ directory loader against the in-memory weights it was written from, and
the GGUF container parser against a file laid out by hand from the GGUF v3 spec (every
metadata value type, alignment padding, Q4_K / F32 / F16 tensors). GPU tests: a model loaded
from a directory decodes the same tokens as the same weights passed in memory (tied and untied
heads; the untied one also against the oracle), and a Q4_K tensor read from a GGUF file
multiplies as the oracle does."""
import json
import os
import struct

import numpy as np
import pytest

from oracle import decode, q4k
from webpytorch_amd import checkpoint, synth

SMALL = dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048, gs=128, bits=4)


# ---- writers (test side) --------------------------------------------------------------------

def _hf_tensors(w, tie):
    """AutoGPTQ / HuggingFace tensor names of a synth.decoder_weights model."""
    t = {}

    def put(name, d):
        t[name + ".qweight"] = np.asarray(d["qweight"], np.int32)
        t[name + ".qzeros"] = np.asarray(d["qzeros"], np.int32)
        t[name + ".scales"] = np.asarray(d["scales"], np.float16)
        t[name + ".g_idx"] = (np.arange(d["qweight"].shape[0] * 8) // w["cfg"]["gs"]).astype(np.int32)
        if d.get("bias") is not None:
            t[name + ".bias"] = np.asarray(d["bias"], np.float16)
    for i, lay in enumerate(w["layers"]):
        p = "model.layers.%d." % i
        for nm, hf in (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
                       ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
                       ("down", "mlp.down_proj")):
            if nm in lay:
                put(p + hf, lay[nm])
        if lay.get("moe"):
            put(p + "mlp.gate", lay["moe"]["router"])
            for e, ex in enumerate(lay["moe"]["experts"]):
                for nm in ("gate", "up", "down"):
                    put(p + "mlp.experts.%d.%s_proj" % (e, nm), ex[nm])
        for key, nm in (("qn", "self_attn.q_norm.weight"), ("kn", "self_attn.k_norm.weight")):
            if lay.get(key) is not None:
                t[p + nm] = np.asarray(lay[key], np.float16)
        t[p + "input_layernorm.weight"] = np.asarray(lay["in_ln"], np.float16)
        t[p + "post_attention_layernorm.weight"] = np.asarray(lay["post_ln"], np.float16)
    t["model.embed_tokens.weight"] = np.asarray(w["embed"], np.float16)
    t["model.norm.weight"] = np.asarray(w["final_norm"], np.float16)
    if not tie:
        t["lm_head.weight"] = np.asarray(w["head"], np.float16)
    return t


def write_gptq_dir(path, w, tie=True, shards=1, declared=4096):
    """An AutoGPTQ model directory written with the safetensors package."""
    from safetensors.numpy import save_file
    c = w["cfg"]
    cfg = {"architectures": ["Qwen2ForCausalLM"], "hidden_size": c["H"], "num_hidden_layers": c["L"],
           "num_attention_heads": c["NH"], "num_key_value_heads": c["NKV"], "intermediate_size": c["I"],
           "vocab_size": c["V"], "rms_norm_eps": 1e-6, "rope_theta": 1e6, "tie_word_embeddings": tie,
           "max_position_embeddings": declared,
           "quantization_config": {"bits": c["bits"], "group_size": c["gs"], "desc_act": False}}
    if c.get("n_experts"):
        cfg.update(num_experts=c["n_experts"], num_experts_per_tok=c["top_k"], moe_intermediate_size=c["moe_I"])
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    t = _hf_tensors(w, tie)
    if shards == 1:
        save_file(t, os.path.join(path, "model.safetensors"))
        return
    names = sorted(t)
    wmap = {}
    for s in range(shards):
        fn = "model-%05d-of-%05d.safetensors" % (s + 1, shards)
        part = {n: t[n] for n in names[s::shards]}
        save_file(part, os.path.join(path, fn))
        wmap.update({n: fn for n in part})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wmap}, f)


def _gguf_str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _gguf_kv(key, vtype, value):
    """One metadata pair, encoded per the GGUF spec (written independently of the parser)."""
    fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}

    def enc(t, v):
        if t in fmt:
            return struct.pack(fmt[t], v)
        if t == 7:
            return bytes([1 if v else 0])
        if t == 8:
            return _gguf_str(v)
        at, items = v
        return struct.pack("<IQ", at, len(items)) + b"".join(enc(at, x) for x in items)
    return _gguf_str(key) + struct.pack("<I", vtype) + enc(vtype, value)


def write_gguf(path, kvs, tensors, align=32):
    """A GGUF v3 file: header, metadata, tensor infos, padding to `align`, tensor data (each
    tensor at an `align`-aligned offset). `tensors` is a list of (name, dims innermost first,
    ggml type id, raw bytes)."""
    if align != 32:
        kvs = list(kvs) + [("general.alignment", 4, align)]
    out = bytearray(struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kvs)))
    for k, t, v in kvs:
        out += _gguf_kv(k, t, v)
    offs, off = [], 0
    for name, dims, ttype, raw in tensors:
        offs.append(off)
        off = (off + len(raw) + align - 1) // align * align
    for (name, dims, ttype, raw), o in zip(tensors, offs):
        out += _gguf_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ttype, o)
    start = (len(out) + align - 1) // align * align
    out += b"\0" * (start - len(out))
    for (name, dims, ttype, raw), o in zip(tensors, offs):
        out += b"\0" * (start + o - len(out)) + raw
    with open(path, "wb") as f:
        f.write(bytes(out))
    return start, offs


# ---- safetensors -----------------------------------------------------------------------------

@pytest.mark.parametrize("shards", [1, 3])
def test_safetensors_reader_against_the_library(tmp_path, shards):
    w = synth.decoder_weights(3, **dict(SMALL, V=128))
    write_gptq_dir(str(tmp_path), w, shards=shards)
    t = _hf_tensors(w, True)
    st = checkpoint.SafetensorsDir(str(tmp_path))
    assert sorted(st.names()) == sorted(t)
    for n, a in t.items():
        got = st.array(n)
        assert got.shape == a.shape
        if a.dtype == np.int32:
            assert got.dtype == np.int32 and np.array_equal(got, a)
        else:  # F16 widens to fp32 exactly
            assert got.dtype == np.float32 and np.array_equal(got, a.astype(np.float32))
            assert np.array_equal(st.array(n, keep_f16=True), a)


def test_safetensors_bf16_f32_and_row_blocks(tmp_path):
    """A file laid out by hand: BF16 widens by a 16-bit shift; row-block fp16 reads of F32 and
    BF16 tables equal whole-table conversion for any block size."""
    g = np.random.default_rng(0)
    f32 = g.standard_normal((37, 24)).astype(np.float32)
    bf = (g.standard_normal((9, 16)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    hdr = {"__metadata__": {"format": "pt"},
           "a": {"dtype": "F32", "shape": [37, 24], "data_offsets": [0, f32.nbytes]},
           "b": {"dtype": "BF16", "shape": [9, 16], "data_offsets": [f32.nbytes, f32.nbytes + bf.nbytes]}}
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    with open(tmp_path / "model.safetensors", "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + f32.tobytes() + bf.tobytes())
    st = checkpoint.SafetensorsDir(str(tmp_path))
    assert sorted(st.names()) == ["a", "b"]
    assert np.array_equal(st.array("a"), f32)
    want_b = (bf.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(st.array("b"), want_b)
    for cb in (1, 100, 24 * 4 * 5, 1 << 20):
        assert np.array_equal(st.rows_f16("a", chunk_bytes=cb), f32.astype(np.float16))
        assert np.array_equal(st.rows_f16("b", chunk_bytes=cb), want_b.astype(np.float16))
    with pytest.raises(KeyError):
        st.array("missing")


def test_gptq_weights_round_trip(tmp_path):
    w = synth.decoder_weights(4, **SMALL)
    w["head"] = (np.random.default_rng(1).standard_normal((SMALL["V"], SMALL["H"])) * 0.02).astype(np.float16)
    write_gptq_dir(str(tmp_path), w, tie=False, shards=2, declared=32768)
    got, declared = checkpoint.gptq_weights(str(tmp_path))
    assert declared == 32768
    c = got["cfg"]
    assert {k: c[k] for k in SMALL} == SMALL and c["eps"] == 1e-6 and c["theta"] == 1e6
    for lay_w, lay_g in zip(w["layers"], got["layers"]):
        for nm in ("q", "k", "v", "o", "gate", "up", "down"):
            assert np.array_equal(lay_g[nm]["qweight"], lay_w[nm]["qweight"])
            assert np.array_equal(lay_g[nm]["qzeros"], lay_w[nm]["qzeros"])
            assert lay_g[nm]["scales"].dtype == np.float16
            assert np.array_equal(lay_g[nm]["scales"], lay_w[nm]["scales"])
            if lay_w[nm].get("bias") is not None:
                assert np.array_equal(lay_g[nm]["bias"], np.asarray(lay_w[nm]["bias"], np.float32))
            else:
                assert "bias" not in lay_g[nm]
        assert np.array_equal(lay_g["in_ln"], np.asarray(lay_w["in_ln"], np.float32))
    assert got["embed"].dtype == np.float16 and np.array_equal(got["embed"], w["embed"])
    assert np.array_equal(got["head"], w["head"])


def test_gptq_config_contract(tmp_path):
    # the context length: request > declared > 2048, capped by the 2 GiB KV budget, >= 512
    assert checkpoint.auto_lmax(100, 4096, 24, 2, 64) == 100
    assert checkpoint.auto_lmax(None, 4096, 24, 2, 64) == 4096
    assert checkpoint.auto_lmax(None, None, 24, 2, 64) == 2048
    assert checkpoint.auto_lmax(None, 10 ** 7, 24, 2, 64) == (2 << 30) // (2 * 24 * 2 * 64 * 4)
    assert checkpoint.auto_lmax(None, 128, 24, 2, 64) == 512
    base = {"hidden_size": 64, "num_hidden_layers": 1, "num_attention_heads": 2, "intermediate_size": 128,
            "vocab_size": 16}
    for extra, err in (({}, ValueError),  # no quantization_config
                       ({"quantization_config": {"bits": 4, "group_size": 64},
                         "layer_types": ["linear_attention"]}, NotImplementedError)):
        with open(tmp_path / "config.json", "w") as f:
            json.dump(dict(base, **extra), f)
        with pytest.raises(err):
            checkpoint.gptq_config(str(tmp_path))
    # sparse MoE fields (`webtorch/llm.py:440-445`)
    with open(tmp_path / "config.json", "w") as f:
        json.dump(dict(base, quantization_config={"bits": 4, "group_size": 64}, num_experts=8, num_experts_per_tok=2,
                       decoder_sparse_step=2, mlp_only_layers=[3]), f)
    c, _, _ = checkpoint.gptq_config(str(tmp_path))
    assert (c["n_experts"], c["top_k"], c["sparse_step"], c["mlp_only"], c["shared_expert"]) == (8, 2, 2, [3], False)
    assert [checkpoint._is_moe_layer(c, i) for i in range(6)] == [False, True, False, False, False, True]
    # nested text_config, head_dim and the defaults
    with open(tmp_path / "config.json", "w") as f:
        json.dump({"text_config": dict(base, head_dim=48), "quantization_config": {"bits": 8, "group_size": 32}}, f)
    c, tie, declared = checkpoint.gptq_config(str(tmp_path))
    assert (c["HD"], c["NKV"], c["bits"], c["gs"], c["theta"], tie, declared) == (48, 2, 8, 32, 10000.0, False, None)


# ---- GGUF ------------------------------------------------------------------------------------

def _gguf_fixture(tmp_path, align):
    W = synth.q4k_layer(9, 512, 3)                           # 3 rows x 2 super-blocks of 144 bytes
    f32 = np.arange(10, dtype=np.float32) * 0.5
    f16 = np.random.default_rng(2).standard_normal((2, 5)).astype(np.float16)
    kvs = [("general.architecture", 8, "qwen2"), ("u8", 0, 200), ("i8", 1, -100), ("u16", 2, 60000),
           ("i16", 3, -30000), ("u32", 4, 4000000000), ("i32", 5, -2000000000), ("f32", 6, 1.5),
           ("bool", 7, True), ("u64", 10, 1 << 40), ("i64", 11, -(1 << 40)), ("f64", 12, 0.1),
           ("qwen2.context_length", 4, 32768), ("tokenizer.ggml.tokens", 9, (8, ["a", "bb", "é"])),
           ("nested", 9, (9, [(5, [1, -2]), (5, [])]))]
    tensors = [("blk.0.ffn_up.weight", [512, 3], 12, W.tobytes()), ("vec", [10], 0, f32.tobytes()),
               ("tab", [5, 2], 1, f16.tobytes())]
    path = str(tmp_path / "m.gguf")
    start, offs = write_gguf(path, kvs, tensors, align=align)
    return path, W, f32, f16, kvs, start, offs


@pytest.mark.parametrize("align", [32, 64])
def test_gguf_header_and_tensors(tmp_path, align):
    path, W, f32, f16, kvs, start, offs = _gguf_fixture(tmp_path, align)
    buf = open(path, "rb").read()
    version, meta, infos, ds = checkpoint.parse_header(buf)
    assert version == 3 and ds == start and ds % align == 0
    for k, t, v in kvs:
        if t == 9:
            v = v[1] if k != "nested" else [x[1] for x in v[1]]
        if t == 6:
            v = np.float32(v)
        assert meta[k] == v, k
    assert [i["name"] for i in infos] == ["blk.0.ffn_up.weight", "vec", "tab"]
    assert [i["offset"] for i in infos] == offs and [i["type"] for i in infos] == [12, 0, 1]
    g = checkpoint.GGUFFile(path, first_read=64)  # the header read grows until it parses
    assert g.shape("blk.0.ffn_up.weight") == (3, 512) and g.type_name("blk.0.ffn_up.weight") == "Q4_K"
    assert g.raw("blk.0.ffn_up.weight") == W.tobytes()
    assert np.array_equal(np.frombuffer(g.raw("vec"), np.float32), f32)
    assert np.array_equal(np.frombuffer(g.raw("tab"), np.float16).reshape(g.shape("tab")), f16)
    with pytest.raises(EOFError):
        checkpoint.parse_header(buf[:ds - align])
    with pytest.raises(ValueError):
        checkpoint.parse_header(b"GGML" + buf[4:])


def test_gguf_tensor_sizes():
    assert checkpoint.tensor_nbytes("Q4_K", 4096) == 16 * 144
    assert checkpoint.tensor_nbytes(14, 512) == 2 * 210          # Q6_K
    assert checkpoint.tensor_nbytes("Q8_0", 64) == 2 * 34
    assert checkpoint.tensor_nbytes("F16", 7) == 14 and checkpoint.tensor_nbytes(0, 7) == 28
    with pytest.raises(ValueError):
        checkpoint.tensor_nbytes("Q4_K", 100)
    assert checkpoint.tensor_nbytes(23, 512) == 2 * 136          # IQ4_XS
    assert checkpoint.tensor_nbytes("IQ4_NL", 64) == 2 * 18
    assert checkpoint.tensor_nbytes(16, 512) == 2 * 66           # IQ2_XXS
    assert checkpoint.tensor_nbytes("MXFP4", 64) == 2 * 17
    assert checkpoint.tensor_nbytes("NVFP4", 128) == 2 * 36
    assert checkpoint.tensor_nbytes(29, 256) == 56               # IQ1_M
    with pytest.raises(NotImplementedError):
        checkpoint.tensor_nbytes(15, 256)                         # Q8_K: not a weight type of the format's files


# ---- GPU -------------------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("tie", [True, False])
def test_from_gptq_decodes_as_in_memory_weights(gpu, tmp_path, tie):
    from webpytorch_amd import llm
    w = synth.decoder_weights(14, gaussian=True, **SMALL)
    if not tie:
        w["head"] = (synth.rng(15, "head").standard_normal((SMALL["V"], SMALL["H"])) * 0.02).astype(np.float16)
    write_gptq_dir(str(tmp_path), w, tie=tie, shards=2)
    ids = synth.prompt_ids(14, 16, SMALL["V"])
    a = llm.CausalLM.from_gptq(str(tmp_path), lmax=64)
    b = llm.CausalLM.from_weights(w, lmax=64)
    ta = a.generate(ids, 16).tokens
    assert ta == b.generate(ids, 16).tokens
    if not tie:  # the untied head is the model's own, quantized as the reference does
        want, _ = decode.Qwen2Oracle(w, lmax=64).generate(ids, 16)
        assert ta == want


@pytest.mark.gpu
def test_gguf_q4k_linear_vs_oracle(gpu, tmp_path):
    import torch
    K, N = 1024, 96
    W = synth.q4k_layer(21, K, N)
    path = str(tmp_path / "w.gguf")
    write_gguf(path, [("general.architecture", 8, "llama")],
               [("output_norm.weight", [K], 0, np.ones(K, np.float32).tobytes()),
                ("blk.0.attn_q.weight", [K, N], 12, W.tobytes())])
    g = checkpoint.GGUFFile(path)
    assert g.linear("output_norm.weight") is None                 # 1-D: not a linear
    lin = g.linear("blk.0.attn_q.weight")
    x = synth.activations(21, 2, K, np.float16)
    got = lin(torch.from_numpy(x)).cpu().numpy()
    ref = q4k.q4k_matmul(x, W, K, N)
    assert np.all(np.abs(got - ref) <= 1e-3 + 1e-2 * np.abs(ref))
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-5


# ---- plain fp16 directories: quantize-on-load and the from_pretrained dispatch ----------------

def write_fp16_dir(path, model):
    """A plain fp16 HuggingFace directory of a `synth.fp16_decoder` model."""
    from safetensors.numpy import save_file
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(model["config"], f)
    save_file(model["tensors"], os.path.join(path, "model.safetensors"))


def test_fp16_dir_config_dispatch(tmp_path):
    """A plain directory is not an AutoGPTQ one, so `from_pretrained` takes the quantize-on-load
    branch (`webtorch/_sdk.py:108-113`); the AutoGPTQ directory takes `from_gptq`."""
    m = synth.fp16_decoder(21, **{k: SMALL[k] for k in ("L", "H", "NH", "NKV", "HD", "I", "V")})
    write_fp16_dir(str(tmp_path / "fp16"), m)
    write_gptq_dir(str(tmp_path / "gptq"), synth.decoder_weights(3, **SMALL))
    assert not checkpoint.is_quantized_dir(str(tmp_path / "fp16"))
    assert checkpoint.is_quantized_dir(str(tmp_path / "gptq"))
    with pytest.raises(ValueError, match="already-quantized"):
        checkpoint.fp16_weights(str(tmp_path / "gptq"), 4)
    with pytest.raises(NotImplementedError):
        checkpoint.fp16_weights(str(tmp_path / "fp16"), 3)


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 8])
def test_from_pretrained_quantizes_fp16_dir_like_the_reference(gpu, tmp_path, bits):
    """`AutoModelForCausalLM.from_pretrained(dir, dtype="int4"|"int8")` on a plain fp16
    directory: every linear quantized on the device on load (gs 128, zero offset 0, fp32 scales;
    int8 group-128 asymmetric), bit-exact with the oracle's `_gptq_quantize`, then greedy ids
    identical to the reference's `from_fp16(quantize=bits)` CPU decode (fixture), eager, unfused
    and graph-replayed."""
    import torch
    from webpytorch_amd import llm
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "decode_fp16q_small.npz"))
    sh = dict(zip(["L", "H", "NH", "NKV", "HD", "I", "V"], [int(v) for v in g["shape"]]))
    model = synth.fp16_decoder(int(g["seed"]), **sh)
    write_fp16_dir(str(tmp_path), model)
    m = llm.AutoModelForCausalLM.from_pretrained(str(tmp_path), dtype="int%d" % bits, lmax=int(g["lmax"]))
    assert m.bits == bits and m.gs == 128 and m.layers[0]["qkv"].zoff == 0.0
    assert m.layers[0]["o"].scales.dtype == torch.float32
    # the device quantizer's output equals the oracle's for a loaded projection
    ow = decode.fp16q_weights(model["tensors"], model["config"], bits)
    assert np.array_equal(m.layers[1]["down"].qweight.cpu().numpy(), ow["layers"][1]["down"]["qweight"])
    assert np.array_equal(m.layers[1]["down"].scales.cpu().numpy().view(np.uint32),
                          ow["layers"][1]["down"]["scales"].view(np.uint32))
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    want = [int(t) for t in g["tokens_int%d" % bits]]
    n = int(g["max_new"])
    assert m.generate(ids, n, use_graph=False).tokens == want
    m.fused = False
    assert m.generate(ids, n, use_graph=False).tokens == want
    m.fused = True
    assert m.generate(ids, n).tokens == want


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 8])
def test_from_pretrained_pads_like_the_reference(gpu, tmp_path, bits):
    """A plain fp16 directory whose sizes the quantizer pads -- a dense layer of intermediate 200
    (the down projection's K padded to 256) and a sparse layer of 60 experts (the router's N
    padded to 64 at int4) -- loads with `dtype="int4"|"int8"` and decodes the reference's greedy
    ids (`from_fp16(quantize=bits)` with `_gquant`'s padding, `webtorch/llm.py:843-849`), eager
    and graph-replayed."""
    from test_oracle_moe_decode import pad_moe_model
    from webpytorch_amd import llm
    g, sh, model = pad_moe_model()
    write_fp16_dir(str(tmp_path), model)
    m = llm.AutoModelForCausalLM.from_pretrained(str(tmp_path), dtype="int%d" % bits, lmax=int(g["lmax"]))
    dn, router = m.layers[0]["down"], m.layers[1]["moe"]["router"]
    assert m.padded and not m.fused and (dn.K, dn.Kt) == (256, 200)
    assert (router.N, router.Nt) == ((64, 60) if bits == 4 else (60, 60))
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    want = [int(t) for t in g["tokens_int%d" % bits]]
    n = int(g["max_new"])
    assert m.generate(ids, n, use_graph=False).tokens == want
    assert m.generate(ids, n).tokens == want


@pytest.mark.gpu
def test_from_pretrained_dispatch_and_refusals(gpu, tmp_path):
    from webpytorch_amd import llm
    w = synth.decoder_weights(14, gaussian=True, **SMALL)
    write_gptq_dir(str(tmp_path / "gptq"), w)
    ids = synth.prompt_ids(14, 16, SMALL["V"])
    # an AutoGPTQ directory loads at its stored bits whatever dtype asks for
    for dt in ("auto", "int8"):
        m = llm.AutoModelForCausalLM.from_pretrained(str(tmp_path / "gptq"), dtype=dt, lmax=64)
        assert m.bits == 4 and m.layers[0]["qkv"].zoff == 1.0
    assert m.generate(ids, 8).tokens == llm.CausalLM.from_weights(w, lmax=64).generate(ids, 8).tokens
    model = synth.fp16_decoder(2, **{k: SMALL[k] for k in ("L", "H", "NH", "NKV", "HD", "I", "V")})
    write_fp16_dir(str(tmp_path / "fp16"), model)
    for dt in ("auto", "fp16"):  # unquantized execution is outside the quantized path
        with pytest.raises(NotImplementedError, match="fp16"):
            llm.AutoModelForCausalLM.from_pretrained(str(tmp_path / "fp16"), dtype=dt, lmax=64)
    with pytest.raises(ValueError, match="dtype"):
        llm.AutoModelForCausalLM.from_pretrained(str(tmp_path / "fp16"), dtype="int3")


@pytest.mark.gpu
def test_from_gptq_moe_qknorm_directory(gpu, tmp_path):
    """A Qwen3-MoE-style AutoGPTQ directory (router `mlp.gate`, experts `mlp.experts.{e}.*`,
    `self_attn.{q,k}_norm`) loads into the engine and decodes the reference's greedy ids."""
    from webpytorch_amd import llm
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "decode_moe_qknorm_small.npz"))
    sh = dict(zip(["L", "H", "NH", "NKV", "HD", "I", "V", "gs", "bits"], [int(v) for v in g["shape"]]))
    ne, mi, k, qk = [int(v) for v in g["extra"]]
    w = synth.decoder_weights(int(g["seed"]), gaussian=True, n_experts=ne, moe_I=mi, top_k=k, qk_norm=bool(qk), **sh)
    write_gptq_dir(str(tmp_path), w, shards=2)
    m = llm.CausalLM.from_gptq(str(tmp_path), lmax=int(g["lmax"]))
    assert m.has_moe and m.has_qk_norm and m.pws is None
    ids = synth.prompt_ids(int(g["seed"]), int(g["prompt_len"]), sh["V"])
    assert m.generate(ids, int(g["max_new"])).tokens == [int(t) for t in g["tokens"]]
