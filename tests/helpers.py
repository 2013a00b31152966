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
