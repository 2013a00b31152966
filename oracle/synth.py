"""Seeded synthetic inputs for the five workload configurations.

Test infrastructure only (see ``oracle/__init__.py``).

Generator: ``numpy.random.default_rng(seed)`` (PCG64), float32 standard normals,
drawn in the fixed order x, logits, [routing-bias permutation], W13, W2 (MoE)
or A, B (dense).  Skewed routing (configuration 3) adds
bias_e = -1.1 * ln(rank_e) to every token's logits, rank = a seeded
permutation of 1..E (a Zipf(s=1.1) popularity profile), which leaves some
experts with no tokens.  Quantisation follows ``spec``: per-tensor amax/448
(weights: one scale per expert tensor) or 1x128 activation groups with 128x128
weight blocks.
"""
import numpy as np

from . import spec

# name -> shape parameters (full size, as in BASELINE.json "configs")
CONFIGS = {
    "dense_2048": dict(kind="dense", M=2048, N=2048, K=2048),
    "mixtral": dict(kind="moe", T=4096, H=4096, I=14336, E=8, k=2, block=False, skew=False),
    "dsv3": dict(kind="moe", T=8192, H=7168, I=2048, E=256, k=8, block=True, skew=True),
    "tp_local": dict(kind="dense", M=8192, N=8192, K=2048),
    "decode": dict(kind="moe", T=64, H=4096, I=1536, E=128, k=8, block=True, skew=False),
}


def skew_bias(rng, num_experts, s=1.1):
    rank = rng.permutation(num_experts).astype(np.float32) + np.float32(1.0)
    return (-np.float32(s) * np.log(rank)).astype(np.float32)


def make_dense(M, N, K, seed=0):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((M, K), dtype=np.float32)
    b = rng.standard_normal((N, K), dtype=np.float32)
    a_q, sa = spec.quant_per_tensor(a)
    b_q, sb = spec.quant_per_tensor(b)
    return dict(a_q=a_q, b_q=b_q, sa=sa, sb=sb)


def make_logits(rng, T, E, skew):
    logits = rng.standard_normal((T, E), dtype=np.float32)
    if skew:
        logits = (logits + skew_bias(rng, E)[None, :]).astype(np.float32)
    return logits


def make_moe(T, H, I, E, k, block, skew, seed=0):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H), dtype=np.float32)
    logits = make_logits(rng, T, E, skew)
    w13 = rng.standard_normal((E, 2 * I, H), dtype=np.float32)
    w2 = rng.standard_normal((E, H, I), dtype=np.float32)
    if block:
        x_q, x_s = spec.quant_group_1x128(x)
        w13_q, w13_s = spec.quant_block_128x128(w13)
        w2_q, w2_s = spec.quant_block_128x128(w2)
    else:
        x_q, x_s = spec.quant_per_tensor(x)
        w13_q = np.empty_like(w13, dtype=np.uint8)
        w2_q = np.empty_like(w2, dtype=np.uint8)
        w13_s = np.empty(E, dtype=np.float32)
        w2_s = np.empty(E, dtype=np.float32)
        for e in range(E):
            w13_q[e], w13_s[e] = spec.quant_per_tensor(w13[e])
            w2_q[e], w2_s[e] = spec.quant_per_tensor(w2[e])
    return dict(x_q=x_q, x_scale=x_s, logits=logits, w13_q=w13_q, w13_s=w13_s,
                w2_q=w2_q, w2_s=w2_s, k=k)


def make(name, seed=0, **override):
    cfg = dict(CONFIGS[name])
    cfg.update(override)
    kind = cfg.pop("kind")
    if kind == "dense":
        return make_dense(cfg["M"], cfg["N"], cfg["K"], seed=seed)
    return make_moe(seed=seed, **cfg)
