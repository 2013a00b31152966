"""MX (microscaling) FP8: 1x32 e8m0 block exponents, restated from the reference.

Test infrastructure only (see ``oracle/__init__.py``).

The reference's only CDNA4 block-scaled GEMM is the MXFP8 kernel of
``kernels/cdna4/gemm/mxfp8/MXFP8_4wave/4_wave.cu``.  Restated here:

  * ``e8m0_from_amax`` / ``quant_mx``: ``compute_e8m0_scale`` and the host
    quantisation loop (4_wave.cu:368-373, 395-413; the device
    ``quantize_fp8_kernel`` at :296-321 computes the same): per row and
    32-element K block, s = clamp(floor(log2(amax)) + 127, 0, 254), 0 for an
    all-zero block, and q = e4m3(x * 2^(127 - s)).  floor(log2(amax)) is taken
    exactly (from the binary exponent of amax); the reference evaluates it
    through a float ``log2`` whose rounding can carry an amax just below a power
    of two up to that power (then s is one larger and q one binade smaller).
  * ``pack_scales_iter`` + ``repack_scales_for_mfma``: ``pack_scales_kernel``
    (:323-338) and ``repack_scales_for_mfma_kernel`` (:340-364), the two steps
    that bring the exponents into the scaled MFMA's operand order.
  * ``mx_pack_scales``: this path's one-step packing with rows padded to 64
    (the library's ``hkmoe_mx_pack_scales``); equal to the two steps above when
    the row count is a multiple of 64.
  * ``gemm_mx``: the CPU reference loop (4_wave.cu:466-478; the 256^3 mini-GEMM
    of tests/unit/cdna4/warp/register/tile/mma_scaled.cu:246-258): C[i, j] =
    sum_kb sum_{k in kb} (A_q[i,k] * 2^(sa[i,kb]-127)) * (B_q[j,k] *
    2^(sb[j,kb]-127)), accumulated here in float64 on the dequantised operands.
    Tolerance of the reference's check: |C - C_ref| <= 0.001 * max|C_ref|
    (4_wave.cu:501-506).
"""
import numpy as np

from .fp8 import bf16_round, e4m3_to_f32, f32_to_e4m3

MX_BLOCK = 32
K_STEP = 128  # K elements per packed word (4 blocks)


def e8m0_from_amax(amax):
    """clamp(floor(log2(amax)) + 127, 0, 254), 0 where amax == 0 (uint8)."""
    amax = np.asarray(amax, dtype=np.float32)
    _, e = np.frexp(amax.astype(np.float64))  # amax = f * 2^e, f in [0.5, 1)
    s = np.clip(e.astype(np.int64) - 1 + 127, 0, 254)
    return np.where(amax > 0, s, 0).astype(np.uint8)


def quant_mx(x):
    """x [R, C] fp32 (finite, C % 32 == 0) -> q [R, C] e4m3, s [R, C/32] e8m0."""
    x = np.asarray(x, dtype=np.float32)
    r, c = x.shape
    assert c % MX_BLOCK == 0
    blk = x.reshape(r, c // MX_BLOCK, MX_BLOCK)
    s = e8m0_from_amax(np.max(np.abs(blk), axis=2))
    # exact power-of-two scaling (float64 holds x * 2^(127-s) exactly), then
    # one rounding to e4m3 (values below fp32's normal range round to 0 in
    # e4m3 either way)
    scaled = np.ldexp(blk.astype(np.float64), (127 - s.astype(np.int64))[:, :, None])
    q = f32_to_e4m3(scaled.astype(np.float32)).reshape(r, c)
    return q, s


def dequant_mx(q, s):
    """e4m3 q [R, C] with e8m0 s [R, C/32] -> float64 [R, C]."""
    r, c = q.shape
    v = e4m3_to_f32(q).astype(np.float64).reshape(r, c // MX_BLOCK, MX_BLOCK)
    return np.ldexp(v, (s.astype(np.int64) - 127)[:, :, None]).reshape(r, c)


def pack_scales_iter(s):
    """pack_scales_kernel: s [R, K/32] -> words [K/128, R], byte j of word
    (ki, row) = s[row, 4*ki + j]."""
    s = np.asarray(s, dtype=np.uint8)
    rows, kb = s.shape
    assert kb % 4 == 0
    k_iters = kb // 4
    out = np.zeros((k_iters, rows), dtype=np.uint32)
    for ki in range(k_iters):
        for j in range(4):
            out[ki] |= s[:, 4 * ki + j].astype(np.uint32) << np.uint32(8 * j)
    return out


def repack_scales_for_mfma(words):
    """repack_scales_for_mfma_kernel: words [K/128, dim] -> [K/128, dim];
    byte g of (ki, row) = byte k_sub of words[ki, tile*64 + g*16 + r16] with
    r16 = row % 16, k_sub = (row / 16) % 4, tile = row / 64 (source rows past
    dim contribute 0)."""
    words = np.asarray(words, dtype=np.uint32)
    k_iters, dim = words.shape
    out = np.zeros_like(words)
    row = np.arange(dim)
    r16, k_sub, tile = row % 16, (row // 16) % 4, row // 64
    for g in range(4):
        src = tile * 64 + g * 16 + r16
        ok = src < dim
        b = (words[:, np.where(ok, src, 0)] >> (8 * k_sub).astype(np.uint32)) & np.uint32(0xFF)
        out |= np.where(ok, b, 0).astype(np.uint32) << np.uint32(8 * g)
    return out


def mx_pack_scales(s):
    """One-step packing: s [R, K/32] -> [K/128, R64] (R64 = R rounded up to
    64); word (kt, p) byte g = s[64*(p//64) + 16*g + p%16, 4*kt + (p%64)//16],
    0 for rows >= R."""
    s = np.asarray(s, dtype=np.uint8)
    rows, kb = s.shape
    assert kb % 4 == 0
    r64 = (rows + 63) // 64 * 64
    pad = np.zeros((r64, kb), dtype=np.uint8)
    pad[:rows] = s
    # [tile, g, r16, kt, k_sub] -> [kt, tile, k_sub, r16] with bytes over g
    t = pad.reshape(r64 // 64, 4, 16, kb // 4, 4)
    t = t.transpose(3, 0, 4, 2, 1).astype(np.uint32)  # kt, tile, k_sub, r16, g
    words = t[..., 0] | (t[..., 1] << 8) | (t[..., 2] << 16) | (t[..., 3] << 24)
    return words.reshape(kb // 4, r64)


def gemm_mx(a_q, sa, b_q, sb, out="f32"):
    """C[M, N] = dequant_mx(A) . dequant_mx(B)^T (float64 sum), returned as
    float32 (out="f32") or rounded to bf16 (out="bf16")."""
    c = (dequant_mx(a_q, sa) @ dequant_mx(b_q, sb).T).astype(np.float32)
    return bf16_round(c) if out == "bf16" else c


def make_mx_dense(M, N, K, seed=42, sigma=0.5):
    """Synthetic MX operands in the shape of the reference's harness
    (4_wave.cu:386-388: N(0, 0.5) values, quantised per 1x32 block); numpy
    PCG64 instead of mt19937, so the values differ, the distribution does not."""
    rng = np.random.default_rng(seed)
    a = rng.normal(0.0, sigma, (M, K)).astype(np.float32)
    b = rng.normal(0.0, sigma, (N, K)).astype(np.float32)
    a_q, sa = quant_mx(a)
    b_q, sb = quant_mx(b)
    return dict(a=a, b=b, a_q=a_q, sa=sa, b_q=b_q, sb=sb)


# ----------------------------------------------------------------------------
# MX mixture-of-experts layer (this path's specification; the reference has no
# MoE code).  Routing, permutation, SiLU*up and combine are spec.py's.
# ----------------------------------------------------------------------------
TILE_M = 256


def tile_words_per_step(rows, num_experts):
    """Words per K step of the tile-aligned exponent layouts."""
    return ((rows + TILE_M - 1) // TILE_M + num_experts) * TILE_M


def gather_words(s_rows, offsets, num_experts):
    """Tile-aligned activation words [K/128, ws] from the exponents of the
    expert-ordered rows s_rows [rows, K/32]: M tile m of expert e (first row
    offsets[e] + 256*j) owns words m*256 .. +255; word m*256 + q of step kt holds
    in byte g the exponent of the tile's row 64*(q//64) + 16g + q%16 for block
    4kt + (q%64)//16, 0 past the expert's rows.  Written as loops over tiles
    and bytes, independently of the kernel's index arithmetic."""
    rows, kb = s_rows.shape
    ws = tile_words_per_step(rows, num_experts)
    out = np.zeros((kb // 4, ws), dtype=np.uint32)
    m = 0
    for e in range(num_experts):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        for row0 in range(lo, hi, TILE_M):
            tile = np.zeros((TILE_M, kb), dtype=np.uint32)
            n = min(TILE_M, hi - row0)
            tile[:n] = s_rows[row0:row0 + n]
            for q in range(TILE_M):
                for g in range(4):
                    r = (q // 64) * 64 + 16 * g + q % 16
                    out[:, m * TILE_M + q] |= tile[r, ((q % 64) // 16)::4] << np.uint32(8 * g)
            m += 1
    return out


def pack_weight_words(s, gate_up=0):
    """Weight words [E, N/256, K/128, 256] from e8m0 s [E, N, K/32]: word p of
    (e, nt, kt) holds in byte g the exponent of B-tile row R = 64*(p//64) +
    16g + p%16 (weight row nt*256 + R, or with gate_up = I the gate/up row
    nt*128 + 32*(R//64) + R%32 + ((R//32)%2)*I) for block 4kt + (p%64)//16."""
    s = np.asarray(s, dtype=np.uint8)
    e_n, n, kb = s.shape
    out = np.zeros((e_n, n // 256, kb // 4, 256), dtype=np.uint32)
    for nt in range(n // 256):
        for p in range(256):
            for g in range(4):
                R = (p // 64) * 64 + 16 * g + p % 16
                wrow = (nt * 128 + 32 * (R // 64) + R % 32 + ((R // 32) % 2) * gate_up) if gate_up \
                    else nt * 256 + R
                out[:, nt, :, p] |= s[:, wrow, ((p % 64) // 16)::4].astype(np.uint32) << np.uint32(8 * g)
    return out


def moe_forward_mx(x_q, x_e8m0, logits, w13_q, w13_e8m0, w2_q, w2_e8m0, k, return_all=False):
    """MX layer: route -> permute -> GEMM1 (MX operands) + SiLU*up -> bf16 h ->
    MX requantisation (quant_mx) -> GEMM2 (MX operands) -> bf16 y -> combine."""
    from . import spec
    e_n = w13_q.shape[0]
    idx, w = spec.route_topk(logits, k)
    counts, offsets = spec.expert_counts_offsets(idx, e_n)
    perm, inv = spec.permutation(idx, e_n)
    xp = x_q[perm // k]
    xs = x_e8m0[perm // k]
    rows = xp.shape[0]
    inter = w13_q.shape[1] // 2
    hidden = w2_q.shape[1]
    z = np.zeros((rows, 2 * inter), dtype=np.float32)
    for e in range(e_n):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi > lo:
            z[lo:hi] = (dequant_mx(xp[lo:hi], xs[lo:hi]) @ dequant_mx(w13_q[e], w13_e8m0[e]).T).astype(np.float32)
    h = bf16_round(spec.silu_mul(z[:, :inter], z[:, inter:]))
    hq, hs = quant_mx(h)
    y = np.zeros((rows, hidden), dtype=np.float32)
    for e in range(e_n):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi > lo:
            y[lo:hi] = (dequant_mx(hq[lo:hi], hs[lo:hi]) @ dequant_mx(w2_q[e], w2_e8m0[e]).T).astype(np.float32)
    y = bf16_round(y)
    out_f32 = spec.combine(y, w, inv, rounded=False)
    out = bf16_round(out_f32)
    if return_all:
        return dict(topk_idx=idx, topk_w=w, counts=counts, offsets=offsets, perm=perm, inv_perm=inv,
                    xs=xs, h=h, hq=hq, hs=hs, y=y, out=out, out_f32=out_f32)
    return out


def make_mx_moe(T, H, I, E, k, skew, seed=0):
    """Seeded MX layer inputs: N(0,1) activations and weights quantised by
    quant_mx (weights per expert row), logits as oracle.synth.make_logits."""
    from .synth import make_logits
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    logits = make_logits(rng, T, E, skew)
    w13 = rng.standard_normal((E, 2 * I, H)).astype(np.float32)
    w2 = rng.standard_normal((E, H, I)).astype(np.float32)
    x_q, x_e = quant_mx(x)
    w13_q, w13_e = quant_mx(w13.reshape(E * 2 * I, H))
    w2_q, w2_e = quant_mx(w2.reshape(E * H, I))
    return dict(x_q=x_q, x_e8m0=x_e, logits=logits, k=k,
                w13_q=w13_q.reshape(E, 2 * I, H), w13_e8m0=w13_e.reshape(E, 2 * I, H // 32),
                w2_q=w2_q.reshape(E, H, I), w2_e8m0=w2_e.reshape(E, H, I // 32))
