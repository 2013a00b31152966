"""Per-token brute-force restatement of the MoE layer (small shapes only).

Test infrastructure only (see ``oracle/__init__.py``).

Structurally independent of ``spec.moe_forward``: no histogram, no offsets, no
permutation and no grouped GEMM.  Each token picks its experts with Python's
``sorted`` on (-logit, expert id), and every (token, slot) pair is pushed
through its expert's weights one at a time.  Agreement with ``spec`` therefore
pins the routing order, the expert-contiguous permutation and the
offset/segment bookkeeping of the grouped GEMMs.
"""
import numpy as np

from .fp8 import bf16_round
from .spec import (dequant_act, dequant_weight, quant_group_1x128,
                   quant_per_tensor, silu_mul)


def topk_bruteforce(logits_row, k):
    items = sorted(range(len(logits_row)), key=lambda e: (-float(logits_row[e]), e))
    sel = items[:k]
    vals = [np.float32(logits_row[e]) for e in sel]
    ex = [np.float32(np.exp(np.float32(v - vals[0]))) for v in vals]
    tot = np.float32(0.0)
    for v in ex:
        tot = np.float32(tot + v)
    return sel, [np.float32(v / tot) for v in ex]


def moe_bruteforce(x_q, x_scale, logits, w13_q, w13_s, w2_q, w2_s, k):
    t_n, _ = x_q.shape
    i_n = w13_q.shape[1] // 2
    block = np.asarray(x_scale).ndim == 2
    xs = np.asarray(x_scale, dtype=np.float32)
    routes = [topk_bruteforce(logits[t], k) for t in range(t_n)]
    hrows = {}
    for t in range(t_n):
        xa = dequant_act(x_q[t:t + 1], xs if xs.ndim == 0 else xs[t:t + 1])[0]
        for j, e in enumerate(routes[t][0]):
            w13 = dequant_weight(w13_q[e], np.asarray(w13_s, dtype=np.float32)[e])
            z = (w13 @ xa).astype(np.float32)
            hrows[(t, j)] = bf16_round(silu_mul(z[:i_n], z[i_n:]))
    keys = [(t, j) for t in range(t_n) for j in range(k)]
    hmat = np.stack([hrows[key] for key in keys])  # slot order f = t*k + j
    if block:
        hq, hs = quant_group_1x128(hmat)
    else:
        hq, hs = quant_per_tensor(hmat)
    out = np.zeros((t_n, w2_q.shape[1]), dtype=np.float32)
    for f, (t, j) in enumerate(keys):
        e = routes[t][0][j]
        w2 = dequant_weight(w2_q[e], np.asarray(w2_s, dtype=np.float32)[e])
        ha = dequant_act(hq[f:f + 1], hs if np.ndim(hs) == 0 else hs[f:f + 1])[0]
        y = bf16_round((w2 @ ha).astype(np.float32))
        out[t] = (out[t] + routes[t][1][j] * y).astype(np.float32)
    return bf16_round(out), routes
