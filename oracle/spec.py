"""Frozen CPU specification of the FP8 MoE grouped-GEMM path (numpy).

Test infrastructure only (see ``oracle/__init__.py``).

The reference has no MoE implementation, so everything below except the dense
GEMM semantics is this path's own written specification.  The dense GEMM
follows the reference's CPU checks: C = A . B^T on dequantised operands with an
fp32 accumulator (``kernels/cdna4/gemm/mxfp8/MXFP8_4wave/4_wave.cu:466-478``;
``kernels/cdna3/gemm/fp8fp32/mi300x/8192_256_256_64_32/data_logs/
0613_003858_outputs/test_python.py:39-48``).  Block scales replace the
reference's 1x32 e8m0 exponents (``4_wave.cu:368-373``) with fp32 scales, so a
dequantised element is ``q * s`` exactly as ``a_q * 2^(sa-127)`` is there.

Layouts (row-major, all integers int32, all scales fp32):
  x_q [T, H] e4m3, x_scale: per-tensor () or per 1x128 group [T, H/128]
  w13_q [E, 2I, H] e4m3 (rows 0..I-1 gate, I..2I-1 up),
  w13_scale: per-tensor [E] or per 128x128 block [E, 2I/128, H/128]
  w2_q [E, H, I] e4m3, w2_scale: [E] or [E, H/128, I/128]
  logits [T, E] fp32 -> topk_idx [T, k], topk_w [T, k]
  counts [E], offsets [E+1] (exclusive scan), perm [T*k], inv_perm [T*k]
  h [T*k, I] bf16 -> hq [T*k, I] e4m3, h_scale () or [T*k, I/128]
  y [T*k, H] bf16 -> out [T, H] bf16
"""
import numpy as np

from .fp8 import E4M3_MAX, bf16_round, e4m3_to_f32, f32_to_e4m3

GROUP = 128


# ----------------------------------------------------------------------------
# quantisers
# ----------------------------------------------------------------------------
FLT_MIN = np.float32(2.0 ** -126)


def scale_from_amax(amax):
    """s = max(amax / 448, 2^-126) in fp32, and 1.0 where amax == 0 (all-zero
    block): every scale is a positive normal fp32 number."""
    amax = np.asarray(amax, dtype=np.float32)
    s = np.maximum(amax / np.float32(E4M3_MAX), FLT_MIN)
    return np.where(amax > 0, s, np.float32(1.0)).astype(np.float32)


def quant_per_tensor(x):
    """Per-tensor e4m3: s = amax/448, q = e4m3(x / s) (fp32 division)."""
    x = np.asarray(x, dtype=np.float32)
    s = scale_from_amax(np.max(np.abs(x)) if x.size else np.float32(0))
    return f32_to_e4m3(x / s), np.float32(s)


def quant_group_1x128(x):
    """Per-row 1x128 group scales: x [R, C] -> q [R, C], s [R, C/128]."""
    x = np.asarray(x, dtype=np.float32)
    r, c = x.shape
    assert c % GROUP == 0
    g = x.reshape(r, c // GROUP, GROUP)
    s = scale_from_amax(np.max(np.abs(g), axis=2))
    q = f32_to_e4m3(g / s[:, :, None]).reshape(r, c)
    return q, s


def quant_block_128x128(w):
    """128x128 block scales: w [..., N, K] -> q, s [..., N/128, K/128]."""
    w = np.asarray(w, dtype=np.float32)
    *lead, n, k = w.shape
    assert n % GROUP == 0 and k % GROUP == 0
    b = w.reshape(*lead, n // GROUP, GROUP, k // GROUP, GROUP)
    s = scale_from_amax(np.max(np.abs(b), axis=(-3, -1)))
    q = f32_to_e4m3(b / s[..., :, None, :, None]).reshape(w.shape)
    return q, s


def dequant_per_tensor(q, s):
    return e4m3_to_f32(q) * np.float32(s)


def dequant_group_1x128(q, s):
    r, c = q.shape
    return (e4m3_to_f32(q).reshape(r, c // GROUP, GROUP) * s[:, :, None]).reshape(r, c)


def dequant_block_128x128(q, s):
    *lead, n, k = q.shape
    v = e4m3_to_f32(q).reshape(*lead, n // GROUP, GROUP, k // GROUP, GROUP)
    return (v * s[..., :, None, :, None]).reshape(q.shape)


def dequant_act(q, s):
    s = np.asarray(s, dtype=np.float32)
    return dequant_per_tensor(q, s) if s.ndim == 0 else dequant_group_1x128(q, s)


def dequant_weight(q, s):
    """q [N, K] with s scalar (per-tensor) or [N/128, K/128] (block)."""
    s = np.asarray(s, dtype=np.float32)
    return dequant_per_tensor(q, s) if s.ndim == 0 else dequant_block_128x128(q, s)


# ----------------------------------------------------------------------------
# dense GEMM (configs 1 and 4)
# ----------------------------------------------------------------------------
def gemm_fp8(a_q, b_q, sa, sb, out="bf16"):
    """C[M,N] = (A_q*sa) . (B_q*sb)^T, fp32 accumulate, bf16 RNE (or fp32) out.

    Follows 4_wave.cu:466-478 (dequantise each operand, fp32 accumulate) and
    test_python.py:46 (``A @ B.t()``)."""
    a = dequant_per_tensor(a_q, sa)
    b = dequant_per_tensor(b_q, sb)
    c = (a @ b.T).astype(np.float32)
    return bf16_round(c) if out == "bf16" else c


# ----------------------------------------------------------------------------
# routing
# ----------------------------------------------------------------------------
def route_topk(logits, k):
    """Top-k experts per token and softmax weights over the selected logits.

    Order: descending logit, ties broken by the lower expert id; slot j holds
    the j-th selected expert.  Weights: e_j = exp(l_j - l_0) in fp32 (l_0 is
    the largest selected logit), sum accumulated sequentially j = 0..k-1 in
    fp32, w_j = e_j / sum."""
    logits = np.asarray(logits, dtype=np.float32)
    t, e = logits.shape
    assert 1 <= k <= e
    order = np.argsort(-logits, axis=1, kind="stable")  # stable: lower id first on ties
    idx = order[:, :k].astype(np.int32)
    sel = np.take_along_axis(logits, idx, axis=1)
    ex = np.exp((sel - sel[:, :1]).astype(np.float32)).astype(np.float32)
    tot = np.zeros(t, dtype=np.float32)
    for j in range(k):
        tot = (tot + ex[:, j]).astype(np.float32)
    w = (ex / tot[:, None]).astype(np.float32)
    return idx, w


def expert_counts_offsets(topk_idx, num_experts):
    """counts[e] = #slots routed to e; offsets = exclusive prefix sum (E+1)."""
    flat = np.asarray(topk_idx, dtype=np.int64).ravel()
    counts = np.bincount(flat, minlength=num_experts).astype(np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    return counts, offsets


def permutation(topk_idx, num_experts):
    """Stable counting sort of flat slots f = t*k + j by expert.

    perm[p] = f for the p-th row of the expert-contiguous buffer (experts in
    ascending order, f ascending inside an expert); inv_perm[f] = p."""
    flat = np.asarray(topk_idx, dtype=np.int64).ravel()
    perm = np.argsort(flat, kind="stable").astype(np.int32)
    inv = np.empty_like(perm)
    inv[perm] = np.arange(perm.size, dtype=np.int32)
    return perm, inv


def permute_rows(x_q, x_scale, perm, k):
    """Gather token rows into expert-contiguous order: row p <- token perm[p]//k."""
    tok = perm.astype(np.int64) // k
    xp = x_q[tok]
    xs = np.asarray(x_scale, dtype=np.float32)
    xps = xs if xs.ndim == 0 else xs[tok]
    return xp, xps


# ----------------------------------------------------------------------------
# grouped GEMMs, epilogue, requantisation, combine
# ----------------------------------------------------------------------------
def silu_mul(g, u):
    """SiLU(g) * u in fp32 with silu(g) = g / (1 + exp(-g))."""
    g = np.asarray(g, dtype=np.float32)
    u = np.asarray(u, dtype=np.float32)
    with np.errstate(over="ignore"):
        sg = (g / (np.float32(1.0) + np.exp(-g))).astype(np.float32)
    return (sg * u).astype(np.float32)


def grouped_gemm(xp, xps, w_q, w_s, offsets):
    """fp32 Y[p] = deq(xp[p]) . deq(W[e])^T for every row p of expert e."""
    e_n = w_q.shape[0]
    n = w_q.shape[1]
    y = np.zeros((xp.shape[0], n), dtype=np.float32)
    xps = np.asarray(xps, dtype=np.float32)
    for e in range(e_n):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi == lo:
            continue
        xa = dequant_act(xp[lo:hi], xps if xps.ndim == 0 else xps[lo:hi])
        wd = dequant_weight(w_q[e], np.asarray(w_s, dtype=np.float32)[e])
        y[lo:hi] = xa @ wd.T
    return y


def gemm1_silu(xp, xps, w13_q, w13_s, offsets, rounded=True):
    """GEMM1 [rows, H] x [2I, H]^T -> h = bf16(SiLU(gate) * up) [rows, I]
    (``rounded=False``: the fp32 value before the bf16 store)."""
    z = grouped_gemm(xp, xps, w13_q, w13_s, offsets)
    i = w13_q.shape[1] // 2
    h = silu_mul(z[:, :i], z[:, i:])
    return bf16_round(h) if rounded else h


def requant(h, block_scaled):
    """Intermediate requantisation: bf16 h -> e4m3 with per-tensor scale
    (amax over the whole [T*k, I] tensor) or 1x128 group scales."""
    return quant_group_1x128(h) if block_scaled else quant_per_tensor(h)


def gemm2(hq, hs, w2_q, w2_s, offsets, rounded=True):
    """GEMM2 [rows, I] x [H, I]^T -> y = bf16 [rows, H] (``rounded=False``:
    fp32)."""
    y = grouped_gemm(hq, hs, w2_q, w2_s, offsets)
    return bf16_round(y) if rounded else y


def combine(y, topk_w, inv_perm, rounded=True):
    """out[t] = bf16( sum_{j=0..k-1} w[t,j] * y[inv_perm[t*k+j]] ), fp32 acc in
    slot order.  ``rounded=False`` returns the fp32 sum before the bf16 store
    (the value the path's error bound is measured against)."""
    t, k = topk_w.shape
    acc = np.zeros((t, y.shape[1]), dtype=np.float32)
    inv = inv_perm.reshape(t, k)
    for j in range(k):
        acc = (acc + topk_w[:, j:j + 1] * y[inv[:, j]]).astype(np.float32)
    return bf16_round(acc) if rounded else acc


def moe_forward(x_q, x_scale, logits, w13_q, w13_s, w2_q, w2_s, k, return_all=False):
    """Whole layer: route -> permute -> GEMM1+SiLU*up -> requant -> GEMM2 ->
    combine.  Block-scaled iff x_scale is 2-D."""
    e_n = w13_q.shape[0]
    block = np.asarray(x_scale).ndim == 2
    idx, w = route_topk(logits, k)
    counts, offsets = expert_counts_offsets(idx, e_n)
    perm, inv = permutation(idx, e_n)
    xp, xps = permute_rows(x_q, x_scale, perm, k)
    h = gemm1_silu(xp, xps, w13_q, w13_s, offsets)
    hq, hs = requant(h, block)
    y = gemm2(hq, hs, w2_q, w2_s, offsets)
    out_f32 = combine(y, w, inv, rounded=False)
    out = bf16_round(out_f32)
    if return_all:
        return dict(topk_idx=idx, topk_w=w, counts=counts, offsets=offsets,
                    perm=perm, inv_perm=inv, xp=xp, xps=xps, h=h, hq=hq, hs=hs,
                    y=y, out=out, out_f32=out_f32)
    return out


def rel_err(got, ref):
    """max|got - ref| / max|ref| (the path's error measure)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.max(np.abs(ref)) if ref.size else 0.0
    if den == 0:
        return float(np.max(np.abs(got))) if got.size else 0.0
    return float(np.max(np.abs(got - ref)) / den)
