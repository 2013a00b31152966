"""Shared test helpers: numpy <-> torch moves for e4m3 bytes and bf16 bits."""
import numpy as np
import torch

from oracle import fp8

F8 = torch.float8_e4m3fn


def to_f8(q_np, dev="cuda"):
    return torch.from_numpy(np.ascontiguousarray(q_np, dtype=np.uint8)).view(F8).to(dev)


def to_f32(a, dev="cuda"):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def to_i32(a, dev="cuda"):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)


def f8_np(t):
    return t.detach().view(torch.uint8).cpu().numpy()


def bf16_np(t):
    """bf16 tensor -> float32 numpy (exact)."""
    return t.detach().float().cpu().numpy()


def moe_inputs_to_gpu(d, dev="cuda"):
    block = np.asarray(d["x_scale"]).ndim == 2
    xs = to_f32(d["x_scale"] if block else np.array([d["x_scale"]], np.float32), dev)
    return dict(x_q=to_f8(d["x_q"], dev), x_scale=xs, logits=to_f32(d["logits"], dev),
                w13_q=to_f8(d["w13_q"], dev), w13_scale=to_f32(d["w13_s"], dev),
                w2_q=to_f8(d["w2_q"], dev), w2_scale=to_f32(d["w2_s"], dev), top_k=int(d["k"]))


def rel_err(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref).max() if ref.size else 0.0
    return float(np.abs(got - ref).max() / den) if den > 0 else float(np.abs(got).max(initial=0.0))


def sampled_layer_reference(tokens, topk_idx, topk_w, x_q, x_s, w13_q, w13_s, w2_q, w2_s, block,
                            h_scale=None):
    """The oracle's layer output (fp32, before the bf16 store) for a few tokens,
    computed per token without permutation or grouped GEMMs: for each slot j of
    token t, expert e = topk_idx[t, j]: h = bf16(SiLU(gate) * up) of the
    dequantised row, requantised (1x128 groups, or the given per-tensor scale),
    y = bf16(h . W2[e]^T), and out[t] = sum_j w[t, j] * y_j in slot order (fp32).

    x_q / x_s: the sampled tokens' e4m3 rows and scales (numpy); w13_q / w2_q
    (and w13_s / w2_s): callables e -> numpy arrays of expert e, so only the
    experts the sampled tokens use are fetched, each once."""
    from oracle import spec
    n = len(tokens)
    k = topk_idx.shape[1]
    xa = spec.dequant_act(x_q, x_s)
    ys = {}
    pairs = {}
    for r, t in enumerate(tokens):
        for j in range(k):
            pairs.setdefault(int(topk_idx[t, j]), []).append((r, j))
    for e, lst in pairs.items():
        w13 = spec.dequant_weight(w13_q(e), w13_s(e))
        w2 = spec.dequant_weight(w2_q(e), w2_s(e))
        inter = w13.shape[0] // 2
        rows = np.array([r for r, _ in lst])
        z = (xa[rows] @ w13.T).astype(np.float32)
        h = spec.bf16_round(spec.silu_mul(z[:, :inter], z[:, inter:]))
        if block:
            hq, hs = spec.quant_group_1x128(h)
        else:
            hs = np.float32(h_scale)
            hq = fp8.f32_to_e4m3((h / hs).astype(np.float32))
        y = spec.bf16_round((spec.dequant_act(hq, hs) @ w2.T).astype(np.float32))
        for q, (r, j) in enumerate(lst):
            ys[(r, j)] = y[q]
    out = np.zeros((n, xa.shape[1]), np.float32)
    for j in range(k):
        for r, t in enumerate(tokens):
            out[r] = (out[r] + topk_w[t, j] * ys[(r, j)]).astype(np.float32)
    return out
