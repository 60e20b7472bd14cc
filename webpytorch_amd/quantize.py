"""Streaming quantizer to the AutoGPTQ safetensors format, on MI355X (`webtorch/quantize.py`).

`stream_quantize` keeps the reference's IO-free contract (`webtorch/quantize.py:108-150`): the
caller supplies async `read_tensor(name) -> ndarray`, `has_tensor(name) -> bool` and
`write_shard(filename, {name: ndarray})`; one input tensor is read, quantized, packed and
added to the current output shard, which is written once it reaches `shard_bytes`; neither the
fp16 model nor the quantized one is ever whole in host memory. The quantization runs on the
device (`miq_gptq_quantize`, bit-exact with `_gptq_quantize`, which computes the same codes as
the reference's `_quantize_raw`) and yields the AutoGPTQ code words (codes packed along K) and
scales (stored as fp16); the zero words, a few KB per tensor, are rewritten on the host to
AutoGPTQ's stored (zp - 1) & mask (`_pack_autogptq`), with g_idx = row // group. `quantize(src_dir, dst_dir, config)` is the local-directory convenience
(`webtorch/quantize.py:153-180`): reads an HF safetensors directory, writes the shards, the
index and a config.json with `quantization_config`.
"""
import asyncio
import inspect
import json
import os

import numpy as np
import torch

from . import core


def _default_pred(name):
    return name.endswith(".weight") and (name.endswith("_proj.weight") or name == "lm_head.weight")


def pack_autogptq_device(W_out_in, bits=4, group_size=128):
    """(out, in) float weight -> AutoGPTQ (qweight (Kp/per, Np) int32, qzeros (G, Np/per) int32,
    scales (G, Np) fp16, g_idx (Kp,) int32) as host arrays: K padded to the group size and N to
    the pack width with zeros (`_quantize_raw`, `webtorch/quantize.py:78-94`), quantized on the
    device, zeros stored as (zp - 1) & mask (`_pack_autogptq`, `webtorch/quantize.py:96-106`)."""
    W = W_out_in if isinstance(W_out_in, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(W_out_in))
    W = W.to(core.device())
    if W.dtype not in (torch.float16, torch.float32):
        W = W.float()
    N, K = int(W.shape[0]), int(W.shape[1])
    per, mask = 32 // bits, (1 << bits) - 1
    Kp, Np = K + (-K) % group_size, N + (-N) % per
    if Kp != K or Np != N:
        W = torch.nn.functional.pad(W.float(), (0, Kp - K, 0, Np - N))
    qw, qz, sc, _, _ = core.gptq_quantize(W.contiguous(), group_size, bits, from_out_in=True)
    # zeros (G, Np / per words, a few KB): unpack along N, store (zp - 1) & mask, repack
    z = qz.cpu().numpy().view(np.uint32)
    qzeros = np.zeros_like(z)
    for j in range(per):
        qzeros |= (((z >> np.uint32(j * bits)) & np.uint32(mask)) - np.uint32(1) & np.uint32(mask)) << np.uint32(j * bits)
    g_idx = np.arange(Kp, dtype=np.int32) // group_size
    return qw.cpu().numpy(), qzeros.view(np.int32), sc.to(torch.float16).cpu().numpy(), g_idx


async def _maybe(v):
    return (await v) if inspect.isawaitable(v) else v


async def stream_quantize(read_tensor, has_tensor, tensor_names, write_shard, bits=4, group_size=128,
                          shard_bytes=512 << 20, quantize_pred=None):
    """IO-free streaming quantizer with the reference's signature and manifest
    (`stream_quantize`, `webtorch/quantize.py:108-150`). `quantize_pred(name)` picks the weights to
    quantize (default: `*_proj.weight` and `lm_head.weight`); the other tensors are stored as
    fp16. Callbacks may be async or plain functions. Returns {weight_map, shards, nq,
    quantization_config}."""
    if quantize_pred is None:
        quantize_pred = _default_pred
    shard, size, wmap, shards = {}, 0, {}, []

    async def flush():
        nonlocal shard, size
        if not shard:
            return
        fn = "model-%05d.safetensors" % (len(shards) + 1)
        await _maybe(write_shard(fn, shard))
        for k in shard:
            wmap[k] = fn
        shards.append(fn)
        shard, size = {}, 0

    async def add(name, arr):
        nonlocal size
        shard[name] = arr
        size += arr.nbytes
        if size >= shard_bytes:
            await flush()

    nq = 0
    for name in tensor_names:
        if quantize_pred(name):
            W = await _maybe(read_tensor(name))
            qw, qz, sc, gidx = pack_autogptq_device(W, bits, group_size)
            del W
            base = name[:-len(".weight")]
            await add(base + ".qweight", qw)
            await add(base + ".qzeros", qz)
            await add(base + ".scales", sc)
            await add(base + ".g_idx", gidx)
            if await _maybe(has_tensor(base + ".bias")):
                await add(base + ".bias", np.asarray(await _maybe(read_tensor(base + ".bias"))).astype(np.float16))
            nq += 1
        else:
            await add(name, np.asarray(await _maybe(read_tensor(name))).astype(np.float16))
    await flush()
    return {"weight_map": wmap, "shards": shards, "nq": nq,
            "quantization_config": {"bits": bits, "group_size": group_size, "desc_act": False, "sym": False,
                                    "quant_method": "gptq"}}


def quantize(src, dst, config=None, bits=4, group_size=128, shard_bytes=512 << 20, names=None,
             quantize_pred=None):
    """Quantize a local HF safetensors directory `src` into an AutoGPTQ directory `dst`
    (`quantize`, `webtorch/quantize.py:153-180`, for local paths): shards, the index and
    config.json (`config` dict, else src/config.json) with `quantization_config`. Returns the
    manifest."""
    from safetensors.numpy import save_file

    from . import checkpoint
    st = checkpoint.SafetensorsDir(src)
    os.makedirs(dst, exist_ok=True)

    def read(name):
        return st.array(name)  # fp32 (F16 / BF16 widen exactly)

    def write(fn, tensors):
        save_file({k: np.ascontiguousarray(v) for k, v in tensors.items()}, os.path.join(dst, fn))

    manifest = asyncio.run(stream_quantize(read, lambda n: n in st, names or sorted(st.names()), write, bits,
                                           group_size, shard_bytes, quantize_pred))
    with open(os.path.join(dst, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": manifest["weight_map"]}, f)
    cfg = dict(config if config is not None else checkpoint.read_config(src))
    cfg["quantization_config"] = manifest["quantization_config"]
    with open(os.path.join(dst, "config.json"), "w") as f:
        json.dump(cfg, f)
    return manifest
