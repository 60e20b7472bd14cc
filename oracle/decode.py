"""CPU greedy decode of a Qwen2-shaped int4 model (test infrastructure only; see
`oracle/__init__.py`).

Follows the reference's growing-cache forward: `CausalLM._kv_forward` (`webtorch/llm.py:
1619-1636`) with `KVCache.attn` (`webtorch/_core.py:1543-1596`), `gqa_attention`
(`_core.py:1319-1340`), the numpy `softmax` (`_core.py:1764-1787`), RMSNorm as an
expression (`llm.py:1260-1268`), HF rotate-half RoPE with float64 angles (`llm.py:1270-1304`),
SwiGLU (`llm.py:1489-1496`, `silu` `_core.py:503-504`), the tied head re-quantized with
`_gptq_quantize` in 4096-row blocks (`llm.py:594-602`) and greedy `argmax` (`llm.py:1336`).
`generate` with no end token yields the prefill's token then one per decode step
(`llm.py:1775-1787`).

A layer given as {"W": fp32 (out, in)[, "bias"]} instead of GPTQ tensors is multiplied in
float32 as given: the reference's native GGUF layers compute x @ dequant(W)^T
(`GGMLLinear` / `UnquantizedLinear`, `webtorch/_core.py:4377-4406, 4462-4481`), and so does a
model whose weights carry "head_W" (a dense head) or "head_q" (GPTQ head blocks) instead of
re-quantizing the head from the embedding.

Pins: golden token ids written by the reference's own `CausalLM` CPU path at a reduced
shape (`tests/golden/`); every building block is also pinned on its own (RMSNorm, RoPE and
softmax closed forms, `gptq.gptq_matmul_np`).
"""
import math

import numpy as np

from . import gptq


class Qwen2Oracle:
    def __init__(self, weights, lmax=256, head_block=4096):
        c = weights["cfg"]
        self.L, self.H, self.NH, self.NKV, self.HD = c["L"], c["H"], c["NH"], c["NKV"], c["HD"]
        self.V, self.gs, self.bits = c["V"], c["gs"], c["bits"]
        self.eps, self.theta = c.get("eps", 1e-6), c.get("theta", 1e6)
        self.lmax = lmax
        self.layers = weights["layers"]
        self.embed = weights["embed"]                      # (V, H) fp16
        self.final_norm = np.asarray(weights["final_norm"], np.float32)
        if weights.get("head_W") is not None:
            self.head = [{"W": np.asarray(weights["head_W"], np.float32)}]
        elif weights.get("head_q") is not None:
            self.head = list(weights["head_q"])
        else:
            # an untied model quantizes its own fp16 lm_head the same way (`webtorch/llm.py:604-612`)
            head = weights.get("head")
            self.head = self.quantize_head(self.embed if head is None else np.asarray(head, np.float16), head_block)

    def quantize_head(self, emb, blk):
        out = []
        for v0 in range(0, emb.shape[0], blk):
            v1 = min(emb.shape[0], v0 + blk)
            qw, qz, sc, _, _ = gptq.gptq_quantize(
                np.ascontiguousarray(emb[v0:v1].astype(np.float32).T), self.gs, self.bits)
            out.append({"qweight": qw, "qzeros": qz, "scales": sc, "K": self.H, "N": v1 - v0,
                        "gs": self.gs, "bits": self.bits})
        return out

    # ---- building blocks ----
    def rms(self, x, w):
        return (x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + self.eps)) * \
            np.asarray(w, np.float32)

    def lin(self, d, x, zoff=None):
        """AutoGPTQ layers use zero offset 1 (`from_autogptq`); layers quantized on load carry
        their own (0, `_gquant`)."""
        if "W" in d:
            y = np.asarray(x, np.float32) @ np.ascontiguousarray(np.asarray(d["W"], np.float32).T)
        else:
            if zoff is None:
                zoff = d.get("zoff", 1.0)
            x = np.asarray(x, np.float32)
            if d.get("Kt", d["K"]) != d["K"]:  # `QuantizedLinear.forward` pads x to Kp (`_core.py:4450-4451`)
                x = np.pad(x, ((0, 0), (0, d["K"] - d["Kt"])))
            y = gptq.gptq_matmul_np(x, d["qweight"], d["qzeros"], d["scales"], d["K"], d["N"],
                                    d["gs"], d["bits"], zoff)[:, :d.get("Nt", d["N"])]
        b = d.get("bias")
        return y if b is None else y + np.asarray(b, np.float32)

    def rope_tables(self, pos, T):
        inv = 1.0 / (self.theta ** (np.arange(0, self.HD, 2, dtype=np.float64) / self.HD))
        ang = np.arange(pos, pos + T, dtype=np.float64)[:, None] * inv[None, :]
        emb = np.concatenate([ang, ang], -1)
        return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)

    def rot(self, x):
        h = self.HD // 2
        return np.concatenate([x[..., h:] * -1.0, x[..., :h]], axis=-1).astype(np.float32)

    @staticmethod
    def softmax(a):
        m = a.max(axis=-1, keepdims=True)
        e = np.exp(a - m)
        return e / e.sum(axis=-1, keepdims=True)

    @staticmethod
    def silu(x):
        return x * (1.0 / (1.0 + np.exp(-x)))

    def attend(self, q, K, V, mask, scale):
        nh, T, hd = q.shape
        nkv, S, _ = K.shape
        rep = nh // nkv
        a = (q.reshape(nkv, rep * T, hd) @ np.ascontiguousarray(K.transpose(0, 2, 1))) * scale
        if mask is not None:
            a = (a.reshape(nkv, rep, T, S) + mask).reshape(nkv, rep * T, S)
        return (self.softmax(a) @ V).reshape(nh, T, hd)

    def mlp(self, lay, x):
        """Dense SwiGLU, or the sparse-MoE block through `moe_mlp` when the layer carries "moe"
        (`CausalLM._mlp`, `webtorch/llm.py:1489-1496`). The reference's layer dict names the
        renormalisation flag "norm_topk" while `moe_mlp` reads "norm_topk_prob"
        (`llm.py:523-524`, `lm_engine.py:304`), so the top-k weights are always renormalised."""
        m = lay.get("moe")
        if m is None:
            return self.lin(lay["down"], self.silu(self.lin(lay["gate"], x)) * self.lin(lay["up"], x))
        from . import moe
        experts = [{k: (lambda t, d=d: self.lin(d, t)) for k, d in e.items()} for e in m["experts"]]
        shared = None
        if m.get("shared"):
            shared = {k: (lambda t, d=d: self.lin(d, t)) for k, d in m["shared"].items()}
        sg = m.get("shared_gate")
        return moe.moe_mlp_np(x, self.lin(m["router"], x), experts, m["top_k"], True, shared=shared,
                              shared_gate=None if sg is None else (lambda t: self.lin(sg, t)))

    # ---- forward ----
    def forward(self, ids, pos, cache):
        """One `_kv_forward` call: T tokens at positions pos.. -> greedy next id, logits."""
        T = len(ids)
        cos, sin = self.rope_tables(pos, T)
        h = np.asarray(self.embed[np.asarray(ids, np.int64)], np.float32)
        scale = 1.0 / math.sqrt(self.HD)
        for i, lay in enumerate(self.layers):
            x = self.rms(h, lay["in_ln"])
            q = self.lin(lay["q"], x).reshape(T, self.NH, self.HD)
            k = self.lin(lay["k"], x).reshape(T, self.NKV, self.HD)
            if lay.get("qn") is not None:  # QK-norm over each head, before RoPE (`llm.py:1516-1517`)
                q = self.rms(q, lay["qn"])
            if lay.get("kn") is not None:
                k = self.rms(k, lay["kn"])
            q, k = q.transpose(1, 0, 2), k.transpose(1, 0, 2)
            v = self.lin(lay["v"], x).reshape(T, self.NKV, self.HD).transpose(1, 0, 2)
            q = q * cos + self.rot(q) * sin
            k = k * cos + self.rot(k) * sin
            if cache[i] is None:
                cache[i] = (np.ascontiguousarray(k), np.ascontiguousarray(v))
            else:
                cache[i] = (np.concatenate([cache[i][0], k], 1), np.concatenate([cache[i][1], v], 1))
            Kc, Vc = cache[i]
            S = Kc.shape[1]
            mask = None
            if T > 1:
                mask = np.triu(np.full((T, S), -1e9, np.float32), 1 + (S - T)).reshape(1, T, S)
            o = self.attend(q, Kc, Vc, mask, scale)
            h = h + self.lin(lay["o"], o.transpose(1, 0, 2).reshape(T, self.NH * self.HD))
            x = self.rms(h, lay["post_ln"])
            h = h + self.mlp(lay, x)
        last = self.rms(h, self.final_norm)[-1:]
        logits = np.concatenate([self.lin(b, last, zoff=0.0) for b in self.head], axis=-1)[0]
        return int(logits.argmax()), logits

    def generate(self, ids, max_new, keep_logits=False):
        """Greedy decode, no end token: returns (token ids, per-step logits or None)."""
        cache = [None] * self.L
        nxt, lg = self.forward(list(ids), 0, cache)
        out, logs, pos = [nxt], [lg] if keep_logits else None, len(ids)
        while len(out) < max_new:
            nxt, lg = self.forward([nxt], pos, cache)
            pos += 1
            out.append(nxt)
            if keep_logits:
                logs.append(lg)
        return out, logs


HF_PROJ = (("q", "self_attn.q_proj"), ("k", "self_attn.k_proj"), ("v", "self_attn.v_proj"),
           ("o", "self_attn.o_proj"), ("gate", "mlp.gate_proj"), ("up", "mlp.up_proj"),
           ("down", "mlp.down_proj"))


def fp16q_weights(tensors, config, bits, gs=128):
    """Oracle weights of a plain fp16 HF model quantized on load, as the reference's
    `from_fp16(quantize=bits)` does (`webtorch/llm.py:1211-1257`): each (out, in) projection read
    as fp32 and quantized by `_gquant` (`webtorch/llm.py:835-853`: `_gptq_quantize` with
    from_out_in, zero offset 0, fp32 scales); the tied head re-quantized from the embedding."""
    c = config
    H, L = c["hidden_size"], c["num_hidden_layers"]
    per = 32 // bits
    kmul = gs if gs % per == 0 else gs * per

    def quant(prefix):
        """`_gquant`: (out, in) fp32 zero-padded to (Np, Kp) -- K to the group multiple, N to the
        pack width (`webtorch/llm.py:843-849`) -- then quantized; the layer keeps Kt / Nt."""
        W = tensors[prefix + ".weight"].astype(np.float32)
        N, K = W.shape
        Kp, Np = K + (-K) % kmul, N + (-N) % per
        qw, qz, sc, _, _ = gptq.gptq_quantize(np.pad(W, ((0, Np - N), (0, Kp - K))), gs, bits, from_out_in=True)
        b = tensors.get(prefix + ".bias")
        return {"qweight": qw, "qzeros": qz, "scales": sc, "K": Kp, "N": Np, "Kt": K, "Nt": N, "gs": gs, "bits": bits,
                "zoff": 0.0, "bias": None if b is None else b.astype(np.float32)}
    n_exp = int(c.get("num_experts", 0) or 0)
    layers = []
    for i in range(L):
        p = "model.layers.%d." % i
        lay = {"in_ln": tensors[p + "input_layernorm.weight"].astype(np.float32),
               "post_ln": tensors[p + "post_attention_layernorm.weight"].astype(np.float32)}
        sparse = n_exp and i not in (c.get("mlp_only_layers") or []) and (i + 1) % int(c.get("decoder_sparse_step", 1)) == 0
        for nm, hf in HF_PROJ:
            if sparse and hf.startswith("mlp."):
                continue
            lay[nm] = quant(p + hf)
        if sparse:  # `_build_layer`'s sparse block (`webtorch/llm.py:522-534`)
            lay["moe"] = {"router": quant(p + "mlp.gate"), "top_k": int(c["num_experts_per_tok"]),
                          "experts": [{n: quant(p + "mlp.experts.%d.%s_proj" % (e, n)) for n in ("gate", "up", "down")}
                                      for e in range(n_exp)]}
        layers.append(lay)
    NH = c["num_attention_heads"]
    cfg = dict(L=L, H=H, NH=NH, NKV=c.get("num_key_value_heads", NH), HD=c.get("head_dim") or H // NH,
               I=c["intermediate_size"], V=c["vocab_size"], gs=gs, bits=bits, eps=c.get("rms_norm_eps", 1e-6),
               theta=c.get("rope_theta", 10000.0))
    return {"layers": layers, "embed": tensors["model.embed_tokens.weight"],
            "final_norm": tensors["model.norm.weight"].astype(np.float32), "cfg": cfg}
