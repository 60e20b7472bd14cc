"""Sparse-MoE MLP oracle (test infrastructure only; see `oracle/__init__.py`).

Follows `moe_mlp` and `_softmax_rows` (`webtorch/lm_engine.py:294-333`): float64 softmax over
all experts, top-k by `argpartition`, renormalised over the k picks, then per expert (in
ascending expert order) `down(silu(gate(x_e)) * up(x_e))` times the float32 routing weight,
accumulated into a float32 output.

Pins: golden vectors written by the reference's own `moe_mlp` (`tests/golden/`), plus the
closed form on tiny instances with tie-free logits (an expert set equal to the identity
reduces the block to sum_j w_j * silu(x) * x).
"""
import numpy as np

from . import gptq


def softmax_rows(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max(1, keepdims=True))
    return e / e.sum(1, keepdims=True)


def route(logits, top_k, norm_topk_prob=True):
    """-> (topk_idx (T, k) int64, topk_w (T, k) float64). Slot order is argpartition's."""
    p = softmax_rows(logits)
    idx = np.argpartition(-p, top_k - 1, axis=1)[:, :top_k]
    w = np.take_along_axis(p, idx, axis=1)
    if norm_topk_prob:
        w = w / w.sum(1, keepdims=True)
    return idx, w


def silu(x):
    return x * (1.0 / (1.0 + np.exp(-x)))


def moe_mlp_np(x, logits, experts, top_k, norm_topk_prob=True, shared=None, shared_gate=None):
    """x (T, H); logits (T, E); experts: list of {gate, up, down} callables (T', K) -> (T', N)
    float32; shared: {gate, up, down} callables or None; shared_gate: callable (T, H) -> (T, 1)
    or None (`webtorch/lm_engine.py:322-328`). Returns (T, H) float32."""
    x = np.asarray(x, np.float32)
    idx, w = route(logits, top_k, norm_topk_prob)
    out = np.zeros((x.shape[0], x.shape[1]), np.float32)
    for e in range(np.asarray(logits).shape[1]):
        rows, slot = np.nonzero(idx == e)
        if rows.size == 0:
            continue
        ex = experts[e]
        xe = x[rows]
        ye = ex["down"](silu(ex["gate"](xe)) * ex["up"](xe))
        ye = ye * w[rows, slot].astype(np.float32).reshape(-1, 1)
        out[rows] = out[rows] + ye
    if shared is not None:
        ys = shared["down"](silu(shared["gate"](x)) * shared["up"](x))
        if shared_gate is not None:
            g = 1.0 / (1.0 + np.exp(-np.asarray(shared_gate(x), np.float32)))
            ys = ys * g
        out = out + ys
    return out


def gptq_linear(d, zoff=1.0, n_out=None):
    """A GPTQ layer dict as a CPU callable x -> x @ W (+ bias), the first n_out columns."""
    def f(t):
        y = gptq.gptq_matmul_np(t, d["qweight"], d["qzeros"], d["scales"], d["K"], d["N"], d["gs"],
                                d["bits"], zoff)
        if d.get("bias") is not None:
            y = y + np.asarray(d["bias"], np.float32)
        return y if n_out is None else y[:, :n_out]
    return f


def gptq_expert(layer_dicts):
    """Wrap AutoGPTQ expert layer dicts as CPU callables (QuantizedLinear with zero bias,
    zero_offset 1, as `QuantizedLinear.from_autogptq` builds them)."""
    return {k: gptq_linear(v) for k, v in layer_dicts.items()}
