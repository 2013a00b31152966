"""The MoE layers of configurations 2, 3 and 5 at full shape, built exactly as
bench.py builds them (bench.make_inputs: x and logits from the path's frozen
PCG64 generator, weights seeded on the device; MoELayer with packed weights and
the library's default narrow split), checked against the oracle.

Every tile (configs 2 and 3), in one pass over the experts:
  * GEMM 1: rows from every 256-row M tile of every expert (a random row, and
    for a partial tile also its last row) and from every narrow expert, against
    the oracle's h of that row (spec.dequant_act / dequant_weight / silu_mul /
    bf16_round).  Per-tensor mode stores bf16 h: max|h - ref| / max|ref| <=
    1e-2.  Block mode stores the requantised h (e4m3 + 1x128 scales): its scale
    within 2^-7 of the oracle's, and every value within the e4m3 rounding of the
    oracle's h: |deq(hq) - h_ref| <= (2^-4 + 2^-7 + 2^-11) |h_ref| + 2^-9 s +
    1e-4 max|h_ref| (half an e4m3 ulp plus one bf16 ulp of h; a wrong row,
    expert or weight block is off by the values' own size).
  * GEMM 2: for every expert e and output column n, the column sum over all of
    e's rows, sum_r y[r, n], against (sum_r deq(hq[r])) . deq(W2[e])[n] in
    float64 (the GPU's own hq as input): |diff| <= 2^-8 sum_r |y[r, n]| +
    2^-12 (sum_r |deq(hq[r])|) . |deq(W2[e])[n]| (bf16 stores and fp32
    accumulation order).
  * sampled tokens chosen to include rows of narrow experts, of partial tiles
    of large experts and of experts of 65-255 rows.

  * routing (top-k ids, offsets, perm, inv_perm): bit-exact vs the oracle on the
    same logits; top-k weights within 1e-6;
  * the one-call layer (the benched hkmoe_moe_forward) == the stepwise layer
    with the same split, bit for bit;
  * sampled tokens: max|out - ref| / max|ref| <= 1e-2 against the oracle's
    per-token layer (helpers.sampled_layer_reference, pinned to
    spec.moe_forward on the CPU);
  * config 5: every active expert is narrow (the all-narrow decode path);
    config 3: both kernels run (narrow experts and 256x256 tiles);
    config 2: per-tensor requantisation scale == scale_from_amax of the GPU's
    own h over all T*k rows, bit for bit.
"""
import numpy as np
import pytest
import torch

import bench
from helpers import bf16_np, f8_np, rel_err, sampled_layer_reference
from oracle import spec

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _np(t):
    return t.detach().cpu().numpy()


def _build(hk, name, seed=0):
    cfg = bench.CONFIGS[name]
    dev = torch.device("cuda:0")
    print(f"config {name}: building inputs {cfg}", flush=True)
    inp = bench.make_inputs(cfg, seed, dev)
    layer = hk.MoELayer(inp["w13_q"], inp["w13_scale"], inp["w2_q"], inp["w2_scale"], inp["top_k"])
    return cfg, inp, layer


def _pick_tokens(steps, counts, k, T, max_rows, seed):
    """Tokens with a slot in a narrow expert (<= max_rows rows), in the partial
    last tile of an expert of more than 256 rows, in an expert of 65..255 rows,
    and a few at random."""
    rng = np.random.default_rng(seed + 7)
    perm = _np(steps["perm"])
    offs = _np(steps["offsets"])
    toks = []
    narrow = np.flatnonzero((counts > 0) & (counts <= max_rows))
    for e in rng.permutation(narrow)[:3]:
        toks.append(int(perm[offs[e]]) // k)
    big = np.flatnonzero((counts > 256) & (counts % 256 != 0))
    for e in rng.permutation(big)[:3]:
        lo = offs[e] + 256 * (counts[e] // 256)
        toks.append(int(perm[rng.integers(lo, offs[e + 1])]) // k)
    mid = np.flatnonzero((counts > max_rows) & (counts < 256))
    for e in rng.permutation(mid)[:2]:
        toks.append(int(perm[offs[e + 1] - 1]) // k)
    toks += [int(t) for t in rng.choice(T, 4, replace=False)]
    return np.array(sorted(set(toks)))


def _deq_weight(q, s):
    """spec.dequant_weight of one expert's weight (a device e4m3 tensor): the
    bytes are decoded by torch's float8_e4m3fn cast (exact, and equal to
    spec.e4m3_to_f32 on all 256 codes: tests/test_oracle.py), about 40x faster
    than the oracle's table lookup on 29M bytes; the scaling is the spec's
    (q * s per 128x128 block, or q * s per tensor)."""
    v = q.float().cpu().numpy()
    s = np.asarray(s, dtype=np.float32)
    n, kk = v.shape
    if s.ndim == 0:
        return v * s
    return (v.reshape(n // 128, 128, kk // 128, 128) * s[:, None, :, None]).reshape(n, kk)


def _every_tile(hk, cfg, inp, steps, counts, block, seed=0):
    """The every-tile checks of GEMM 1 and GEMM 2 (module docstring), one pass
    over the active experts, each expert's weights dequantised once."""
    k, I = cfg["k"], cfg["I"]
    rng = np.random.default_rng(seed + 3)
    perm = _np(steps["perm"])
    offs = _np(steps["offsets"])
    hq = f8_np(steps["hq"])
    hs = _np(steps["hs"])
    y = steps["y"]
    x_q = f8_np(inp["x_q"])
    x_s = _np(inp["x_scale"])
    w13s, w2s = _np(inp["w13_scale"]), _np(inp["w2_scale"])
    h_gpu = bf16_np(steps["h"]) if not block else None
    n_rows = n_tiles = 0
    worst1 = worst2 = 0.0
    for e in np.flatnonzero(counts):
        lo, hi = int(offs[e]), int(offs[e + 1])
        # GEMM 1: rows of every M tile (one segment for a narrow expert)
        rows = []
        for t0 in range(lo, hi, 256):
            t1 = min(t0 + 256, hi)
            rows.append(int(rng.integers(t0, t1)))
            if t1 - t0 < 256:
                rows.append(t1 - 1)
            n_tiles += 1
        rows = np.array(sorted(set(rows)))
        n_rows += len(rows)
        tok = perm[rows] // k
        xa = spec.dequant_act(x_q[tok], x_s[tok] if block else np.float32(x_s[0]))
        w13 = _deq_weight(inp["w13_q"][e], w13s[e])
        if e == int(np.flatnonzero(counts)[0]):  # the decode agrees with the oracle's
            np.testing.assert_array_equal(w13[:128, :128],
                                          spec.dequant_weight(f8_np(inp["w13_q"][e][:128, :128]),
                                                              w13s[e] if w13s[e].ndim == 0 else w13s[e][:1, :1]))
        z = (xa @ w13.T).astype(np.float32)
        del w13
        h_ref = spec.bf16_round(spec.silu_mul(z[:, :I], z[:, I:]))
        if block:
            sc = hs[:, rows].T                                   # [rows, I/128]
            deq = spec.dequant_group_1x128(hq[rows], sc)
            _, s_ref = spec.quant_group_1x128(h_ref)
            assert np.all(np.abs(sc / s_ref - 1.0) <= 2.0 ** -7), (e, rows)
            smax = np.repeat(sc, 128, axis=1)
            # e4m3 rounding of h / s (half an ulp: 2^-4 relative, 2^-10 s in the
            # subnormal range) on top of one bf16 ulp of h (<= 2^-7 relative) from
            # the accumulation order and the hardware exp / reciprocal
            bound = ((2.0 ** -4 + 2.0 ** -7 + 2.0 ** -11) * np.abs(h_ref) + 2.0 ** -9 * smax
                     + 1e-4 * np.abs(h_ref).max(axis=1, keepdims=True))
            ratio = np.abs(deq - h_ref) / bound
            worst1 = max(worst1, float(ratio.max()))
            assert np.all(ratio <= 1.0), (e, rows[np.argmax(ratio.max(axis=1))])
        else:
            err = rel_err(h_gpu[rows], h_ref)
            worst1 = max(worst1, err)
            assert err <= TOL, (e, err)
        # GEMM 2: column sums over all of the expert's rows
        hd = (spec.dequant_group_1x128(hq[lo:hi], hs[:, lo:hi].T) if block
              else spec.dequant_per_tensor(hq[lo:hi], hs[0])).astype(np.float64)
        w2 = _deq_weight(inp["w2_q"][e], w2s[e]).astype(np.float64)
        ye = y[lo:hi].double()
        got = ye.sum(0).cpu().numpy()
        yabs = ye.abs().sum(0).cpu().numpy()
        ref = hd.sum(0) @ w2.T
        acc = np.abs(hd).sum(0) @ np.abs(w2).T
        del w2
        ratio = np.abs(got - ref) / (2.0 ** -8 * yabs + 2.0 ** -12 * acc)
        worst2 = max(worst2, float(ratio.max()))
        assert np.all(ratio <= 1.0), (e, int(np.argmax(ratio)))
    print(f"every tile: {n_tiles} M tiles / segments, {n_rows} GEMM 1 rows, "
          f"{int((counts > 0).sum())} experts' GEMM 2 column sums; worst GEMM 1 "
          f"{'|diff| / bound' if block else 'rel err'} {worst1:.3e}, worst GEMM 2 |diff| / bound {worst2:.3e}",
          flush=True)


def _check(hk, name, n_tokens, seed=0, every_tile=False):
    cfg, inp, layer = _build(hk, name, seed)
    T, E, k = cfg["T"], cfg["E"], cfg["k"]
    out = layer(inp["x_q"], inp["x_scale"], inp["logits"])
    narrow = bench.narrow_setting(inp)
    steps = hk.moe_forward_steps(inp["x_q"], inp["x_scale"], inp["logits"], layer.w13_q, inp["w13_scale"],
                                 layer.w2_q, inp["w2_scale"], k, packed=True, narrow=narrow)
    torch.cuda.synchronize()
    print(f"config {name}: layer done, narrow={narrow}", flush=True)
    assert torch.equal(out.view(torch.int16), steps["out"].view(torch.int16))

    # routing vs the oracle on the same logits
    logits = _np(inp["logits"])
    idx_ref, w_ref = spec.route_topk(logits, k)
    np.testing.assert_array_equal(_np(steps["topk_idx"]), idx_ref)
    assert rel_err(_np(steps["topk_w"]), w_ref) <= 1e-6
    counts_ref, offs_ref = spec.expert_counts_offsets(idx_ref, E)
    np.testing.assert_array_equal(_np(steps["offsets"]), offs_ref)
    p_ref, i_ref = spec.permutation(idx_ref, E)
    np.testing.assert_array_equal(_np(steps["perm"]), p_ref)
    np.testing.assert_array_equal(_np(steps["inv_perm"]), i_ref)

    if every_tile:
        _every_tile(hk, cfg, inp, steps, counts_ref, cfg["block"], seed)
        max_rows = narrow[1] if narrow is not None else 64
        toks = _pick_tokens(steps, counts_ref, k, T, max_rows, seed)
    else:
        # sampled tokens vs the per-token oracle
        toks = np.sort(np.random.default_rng(seed + 1).choice(T, n_tokens, replace=False))
    n_tokens = len(toks)
    sel = torch.from_numpy(toks).cuda()
    block = cfg["block"]
    xq = f8_np(inp["x_q"][sel])
    xs = _np(inp["x_scale"][sel]) if block else np.float32(_np(inp["x_scale"])[0])
    h_scale = None
    if not block:
        # per-tensor requantisation: one scale from the amax of all T*k rows of h
        h_all = bf16_np(steps["h"])
        h_scale = spec.scale_from_amax(np.abs(h_all).max())
        assert _np(steps["hs"])[0] == h_scale
        del h_all
    w13, w2 = inp["w13_q"], inp["w2_q"]
    w13s, w2s = _np(inp["w13_scale"]), _np(inp["w2_scale"])
    ref = sampled_layer_reference(toks, idx_ref, w_ref, xq, xs,
                                  lambda e: f8_np(w13[e]), lambda e: w13s[e],
                                  lambda e: f8_np(w2[e]), lambda e: w2s[e], block, h_scale=h_scale)
    err = rel_err(bf16_np(out[sel]), ref)
    print(f"config {name}: {n_tokens} sampled tokens, rel_err={err:.3e}", flush=True)
    assert err <= TOL
    return cfg, steps, counts_ref, narrow


@pytest.mark.timeout(600)
def test_config3_dsv3_full_shape(hk):
    cfg, steps, counts, narrow = _check(hk, "dsv3", n_tokens=8, every_tile=True)
    assert narrow is not None
    _, max_rows, _ = narrow
    n_narrow = int(((counts > 0) & (counts <= max_rows)).sum())
    assert int(steps["narrow_info"][0]) == n_narrow and n_narrow > 0
    assert (counts > 256).any()        # 256x256 tiles as well
    assert (counts == 0).sum() > 0     # skewed: some experts get no tokens


@pytest.mark.timeout(300)
def test_config5_decode_all_narrow(hk):
    cfg, steps, counts, narrow = _check(hk, "decode", n_tokens=16)
    assert narrow is not None
    active = int((counts > 0).sum())
    assert counts.max() <= narrow[1]
    assert int(steps["narrow_info"][0]) == active   # every active expert is narrow


@pytest.mark.timeout(400)
def test_config2_mixtral_full_shape(hk):
    cfg, steps, counts, narrow = _check(hk, "mixtral", n_tokens=8, every_tile=True)
    assert narrow is None               # per-tensor scales: 256x256 tiles only
    assert (counts > 0).all()
