"""Phase timeline of the persistent decode step (`miq_decode_persistent_trace`).

    python -m webpytorch_amd.pd_trace [--steps N] [--prompt P] [--full]

Builds the random-init Qwen2-0.5B-shaped int4 model the bench uses, prefills a P-token
prompt, runs N traced decode steps (each on a zeroed trace buffer) and prints, for the last
step, the per-layer timeline of each role and its averages over the middle layers:

  * `got`: when a role's workgroups had all their inputs (first .. last workgroup);
  * `st`: when the last of them had published its result;
  * per role, the time from `got` to inputs staged / matrix product done / tile summed /
    published (the marks of `miq_decode_persistent_trace`);
  * per hop, the time from the producers' last publish to the consumers' last `got`.

Times are microseconds of the GPU wall clock (100 MHz), relative to the earliest kernel entry.
Workgroup roles follow the kernel's order: q|k|v tiles, query heads, o tiles, gate|up tiles,
down (tile, K-slice) pairs; the rest take part in the head only.
"""
import argparse
import sys

import numpy as np
import torch

from . import _lib, llm, synth
from .core import ptr, stream_handle


def trace_steps(m, steps):
    """Runs `steps` traced decode steps of model m (prefilled); returns the last step's marks as
    an int64 array [G][L + 2][8] and the step times in ms (CUDA events)."""
    G = m.persistent_grid
    tr = torch.zeros(G * (m.L + 2) * 8, dtype=torch.int64, device="cuda")
    b = m.buf
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    times = []
    for _ in range(steps):
        tr.zero_()
        ev[0].record()
        _lib.call("miq_decode_persistent_trace", ptr(m.layer_table), ptr(m.embed), ptr(m.head.qweight),
                  ptr(m.head.qzeros), ptr(m.head.scales), ptr(m.final_norm), ptr(m.cos_t), ptr(m.sin_t), ptr(m.ids),
                  ptr(m.history), m.lmax, ptr(m.state), ptr(b["logits"]), ptr(m.pws), m.pws.numel(), m.L, m.H, m.NH,
                  m.NKV, m.HD, m.I, m.V, m.lmax, m.gs, m.bits, m.eps, float(m.layers[0]["qkv"].zoff),
                  float(m.head.zoff), ptr(tr), tr.numel(), stream_handle())
        ev[1].record()
        torch.cuda.synchronize()
        times.append(ev[0].elapsed_time(ev[1]))
    if m.persistent_error():
        raise _lib.MiqError("traced step failed with error bits %d" % m.persistent_error())
    return tr.cpu().numpy().reshape(G, m.L + 2, 8).astype(np.int64), times


def role_ranges(m, t):
    nq, na, no, ngu = (m.NH + 2 * m.NKV) * m.HD // 64, m.NH, m.H // 64, 2 * m.I // 64
    o = nq + na + no + ngu
    nd = int(np.count_nonzero(t[o:, 0, 0]))  # down workgroups mark layer 0; head-only ones do not
    edges = np.cumsum([0, nq, na, no, ngu, nd])
    names = ("qkv", "attn", "ored", "gu", "down")
    return {n: np.arange(edges[i], edges[i + 1]) for i, n in enumerate(names)}


def summarize(m, t, full=False, out=sys.stdout):
    roles = role_ranges(m, t)
    t0 = t[:, m.L + 1, 0].min()
    us = lambda x: (np.asarray(x, np.float64) - t0) / 100.0  # noqa: E731  100 MHz ticks -> us
    pr = lambda *a: print(*a, file=out)  # noqa: E731
    pr("kernel entry spread %.2f us, exit %.2f us (%d workgroups, %d layers)" % (
        us(t[:, m.L + 1, 0].max()), us(t[:, m.L + 1, 1].max()), t.shape[0], m.L))
    names = list(roles)
    pr("layer " + " | ".join("%-19s" % ("%s got..  st" % n) for n in names))
    for l in (range(m.L) if full else sorted({1, m.L // 2, m.L - 1})):
        cells = []
        for n in names:
            r = roles[n]
            cells.append("%6.1f..%5.1f %6.1f" % (us(t[r, l, 1].min()), us(t[r, l, 1].max()), us(t[r, l, 2].max())))
        pr("%5d " % l + " | ".join(cells))
    mid = range(1, m.L - 1) if m.L > 2 else range(0, m.L - 1)  # layers with a layer before and after
    stage = {}
    for n in names:
        r = roles[n]
        got = t[np.ix_(r, list(mid))][:, :, 1]
        row = {}
        for k, label in ((3, "staged"), (5, "product"), (4, "summed"), (2, "published")):
            v = t[np.ix_(r, list(mid))][:, :, k]
            if np.all(v > 0):
                row[label] = float(np.mean((v - got) / 100.0))
        stage[n] = row
        pr("%5s after inputs: " % n + "  ".join("%s %.2f" % kv for kv in row.items()))
    # a role's work: its last workgroup's publish minus its last input arrival, per layer
    work = {n: float(np.mean([(t[roles[n], l, 2].max() - t[roles[n], l, 1].max()) / 100.0 for l in mid]))
            for n in names}
    pairs = (("qkv", "attn", 0), ("attn", "ored", 0), ("ored", "gu", 0), ("gu", "down", 0), ("down", "qkv", 1))
    hops = {"%s->%s" % (a, b): float(np.mean([(t[roles[b], l + d, 1].max() - t[roles[a], l, 2].max()) / 100.0
                                              for l in mid])) for a, b, d in pairs}
    period = float(np.mean([(t[roles["qkv"], l + 1, 1].max() - t[roles["qkv"], l, 1].max()) / 100.0 for l in mid]))
    pr("work per layer: " + "  ".join("%s %.2f" % kv for kv in work.items()))
    pr("hops: " + "  ".join("%s %.2f" % kv for kv in hops.items()))
    pr("layer period %.2f us" % period)
    head = t[:, m.L, :]
    pr("head: h(L) received %.1f..%.1f, arg-max published by %.1f; token done %.1f" % (
        us(head[:, 1].min()), us(head[:, 1].max()), us(head[:, 2].max()), us(t[:, m.L + 1, 1].max())))
    return {"stages": stage, "work": work, "hops": hops, "period": period}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--steps", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=64)
    ap.add_argument("--full", action="store_true", help="every layer's timeline")
    a = ap.parse_args(argv)
    m = llm.CausalLM.from_weights(synth.decoder_weights(5, **synth.QWEN2_05B), lmax=256, persistent=True)
    ids = synth.prompt_ids(5, a.prompt, synth.QWEN2_05B["V"])
    m.generate(ids, 1, use_graph=False)
    t, times = trace_steps(m, a.steps)
    print("traced step times (ms): " + " ".join("%.3f" % x for x in times))
    summarize(m, t, a.full)


if __name__ == "__main__":
    main()
