"""The streaming AutoGPTQ writer (`stream_quantize` / `quantize`, `webtorch/quantize.py:108-180`):
every quantized tensor it writes equals the oracle's `_gptq_quantize` codes and scales in the
AutoGPTQ packing (`pack_autogptq`: stored zero (zp - 1) & mask, fp16 scales, g_idx), padding
included; other tensors pass through as fp16; shards split at `shard_bytes` and the manifest maps
every tensor; the directory it writes loads with `from_gptq` and decodes what the CPU oracle
decodes over the same files."""
import asyncio
import json
import os

import numpy as np
import pytest

from oracle import decode, gptq
from test_checkpoint import write_fp16_dir
from webpytorch_amd import synth

pytestmark = pytest.mark.gpu

SH = dict(L=2, H=256, NH=4, NKV=2, HD=64, I=512, V=2048)


def expected_autogptq(W_out_in, bits, gs):
    """The reference's packing of one (out, in) weight, from the oracle quantizer."""
    W = np.asarray(W_out_in, np.float32)
    N, K = W.shape
    per = 32 // bits
    Kp, Np = K + (-K) % gs, N + (-N) % per
    W = np.pad(W, ((0, Np - N), (0, Kp - K)))
    qw, qz, sc, _, _ = gptq.gptq_quantize(W, gs, bits, from_out_in=True)
    codes = gptq.unpack_along_k(qw, bits)
    zp = gptq.unpack_along_n(qz, bits)
    return gptq.pack_autogptq(codes, sc, zp, gs, bits)


@pytest.mark.parametrize("bits", [4, 8])
def test_stream_quantize_packs_like_the_reference(gpu, bits):
    from webpytorch_amd import quantize
    g = np.random.default_rng(bits)
    src = {"a.q_proj.weight": (g.standard_normal((40, 200)) * 0.05).astype(np.float16),  # K, N padded
           "a.q_proj.bias": (g.standard_normal(40) * 0.1).astype(np.float16),
           "b.down_proj.weight": (g.standard_normal((64, 384)) * 0.05).astype(np.float16),
           "norm.weight": (1 + 0.1 * g.standard_normal(64)).astype(np.float16),
           "lm_head.weight": (g.standard_normal((96, 128)) * 0.02).astype(np.float16)}
    # a group whose minimum is 0 stores zero 0 as (0 - 1) & mask, as AutoGPTQ's writer does
    src["b.down_proj.weight"][:, :128] = np.abs(src["b.down_proj.weight"][:, :128])
    shards = {}

    async def read(n):
        return src[n]

    async def has(n):
        return n in src

    async def write(fn, tensors):
        shards[fn] = dict(tensors)

    man = asyncio.run(quantize.stream_quantize(read, has, list(src), write, bits=bits, group_size=128,
                                               shard_bytes=1 << 14))
    assert man["nq"] == 3 and len(man["shards"]) == len(shards) >= 2
    assert man["quantization_config"] == {"bits": bits, "group_size": 128, "desc_act": False, "sym": False,
                                          "quant_method": "gptq"}
    out = {}
    for fn, tensors in shards.items():
        for k, v in tensors.items():
            assert man["weight_map"][k] == fn
            out[k] = v
    for base in ("a.q_proj", "b.down_proj", "lm_head"):
        want = expected_autogptq(src[base + ".weight"], bits, 128)
        for suffix, w in zip((".qweight", ".qzeros", ".scales", ".g_idx"), want):
            got = out[base + suffix]
            assert got.dtype == w.dtype and got.shape == w.shape, (base, suffix)
            assert np.array_equal(got.view(np.uint8), np.ascontiguousarray(w).view(np.uint8)), (base, suffix)
    zs = gptq.unpack_along_n(out["b.down_proj.qzeros"], bits)
    assert (zs[0] == (1 << bits) - 1).any()  # the wrapped stored zero of the non-negative group
    assert np.array_equal(out["a.q_proj.bias"], src["a.q_proj.bias"])
    assert np.array_equal(out["norm.weight"], src["norm.weight"])


def test_quantize_directory_loads_and_decodes_like_the_oracle(gpu, tmp_path):
    import torch
    from safetensors.numpy import load_file

    from webpytorch_amd import llm, quantize
    model = synth.fp16_decoder(31, **SH)
    write_fp16_dir(str(tmp_path / "fp16"), model)
    man = quantize.quantize(str(tmp_path / "fp16"), str(tmp_path / "q4"), bits=4, shard_bytes=1 << 20)
    assert len(man["shards"]) >= 2
    cfg = json.load(open(tmp_path / "q4" / "config.json"))
    assert cfg["quantization_config"]["bits"] == 4 and cfg["hidden_size"] == SH["H"]
    t = {}
    for fn in man["shards"]:
        t.update(load_file(os.path.join(tmp_path / "q4", fn)))
    layers = []
    for i in range(SH["L"]):
        p = "model.layers.%d." % i
        lay = {"in_ln": t[p + "input_layernorm.weight"].astype(np.float32),
               "post_ln": t[p + "post_attention_layernorm.weight"].astype(np.float32)}
        for nm, hf in decode.HF_PROJ:
            qw = t[p + hf + ".qweight"]
            b = t.get(p + hf + ".bias")
            lay[nm] = {"qweight": qw, "qzeros": t[p + hf + ".qzeros"], "scales": t[p + hf + ".scales"].astype(np.float32),
                       "K": qw.shape[0] * 8, "N": qw.shape[1], "gs": 128, "bits": 4, "zoff": 1.0,
                       "bias": None if b is None else b.astype(np.float32)}
        layers.append(lay)
    ow = {"layers": layers, "embed": t["model.embed_tokens.weight"], "final_norm": t["model.norm.weight"].astype(np.float32),
          "cfg": dict(L=SH["L"], H=SH["H"], NH=SH["NH"], NKV=SH["NKV"], HD=SH["HD"], V=SH["V"], gs=128, bits=4,
                      eps=1e-6, theta=1e6)}
    ora = decode.Qwen2Oracle(ow, lmax=64)
    m = llm.CausalLM.from_gptq(str(tmp_path / "q4"), lmax=64)
    ids = synth.prompt_ids(31, 9, SH["V"])
    want, logs = ora.generate(ids, 9, keep_logits=True)
    m.generate(ids, 1, use_graph=False)
    got = [int(m.history[0])]
    for s in range(8):
        np.testing.assert_allclose(m.buf["logits"][0].cpu().numpy(), logs[s], rtol=1e-4,
                                   atol=1e-4 * np.abs(logs[s]).max())
        m._step(1)
        torch.cuda.synchronize()
        got.append(int(m.history[s + 1]))
    checked = 0
    for s, lg in enumerate(logs[:9]):
        top2 = np.sort(lg)[-2:]
        if top2[1] - top2[0] <= 1e-3 * np.abs(lg).max():
            break
        assert got[s] == want[s], (s, got, want)
        checked += 1
    assert checked >= 4
