"""Pins for the CPU oracle (no GPU).

The reference ships no MoE code and no golden vectors for this path, so every
oracle function is pinned here by something independent of its own formula:

  fp8.e4m3_to_f32 / f32_to_e4m3   torch.float8_e4m3fn (library) on all 256 codes
                                  and 1M random values; saturation/NaN/ties closed forms
  fp8.bf16_round                  torch.bfloat16 cast (library, RNE)
  spec.quant_*                    closed forms: amax element -> +-448 exactly,
                                  half-ulp error bound, all-zero group -> scale 1,
                                  FLT_MIN floor
  spec.route_topk                 torch.topk / torch.softmax (library) on tie-free
                                  logits; brute-force Python sort with ties; the
                                  all-equal closed form
  spec.expert_counts_offsets,
  spec.permutation                brute-force Python loops; permutation invariants
  spec.gemm_fp8                   +-1 known-answer test (exact integer sums, as in
                                  cdna3 test_python.py:8-12) and torch.matmul
  spec.silu_mul                   torch.nn.functional.silu (library)
  spec.combine                    brute-force loops
  spec.moe_forward                oracle.brute (per-token restatement without
                                  permutation or grouped GEMM)
  whole oracle                    tests/golden fixtures (frozen outputs)
A final test plants mistakes in the oracle (on the CPU) and checks that these
pins catch them.
"""
import os

import numpy as np
import pytest
import torch

from oracle import brute, fp8, mx, spec, synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ----------------------------------------------------------------------------
# number formats
# ----------------------------------------------------------------------------
def test_e4m3_decode_all_codes_vs_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = fp8.e4m3_to_f32(codes)
    assert np.array_equal(np.isnan(ref), np.isnan(got))
    m = ~np.isnan(ref)
    assert np.array_equal(ref[m].view(np.uint32), got[m].view(np.uint32))  # incl. signed zero


def test_e4m3_encode_vs_torch_random_and_edges():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(1 << 20).astype(np.float32) * np.float32(60),
        rng.standard_normal(1 << 16).astype(np.float32) * np.float32(2 ** -8),   # subnormals
        fp8.E4M3_LUT[:0x7F],                                                   # exact codes
        (fp8.E4M3_LUT[:0x7E] + fp8.E4M3_LUT[1:0x7F]) / 2,                      # ties
        -(fp8.E4M3_LUT[:0x7E] + fp8.E4M3_LUT[1:0x7F]) / 2,
        np.array([0.0, -0.0, 447.9, -447.9, 2 ** -10, -2 ** -10], np.float32),
    ]).astype(np.float32)
    x = x[np.abs(x) < 464]  # torch turns |x| >= 480 into NaN; rounding to 448 below 464
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(fp8.f32_to_e4m3(x), ref)


def test_e4m3_saturation_and_nan():
    x = np.array([448.0, 464.0, 500.0, 1e30, np.inf, -1e30, -np.inf, np.nan, -np.nan], np.float32)
    q = fp8.f32_to_e4m3(x)
    assert list(q[:5]) == [0x7E] * 5
    assert list(q[5:7]) == [0xFE] * 2
    assert (q[7] & 0x7F) == 0x7F and (q[8] & 0x7F) == 0x7F
    assert fp8.e4m3_to_f32(np.uint8(0x7E)) == 448.0
    assert fp8.e4m3_to_f32(np.uint8(0x01)) == 2.0 ** -9


def test_bf16_round_vs_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(1 << 18).astype(np.float32) * np.float32(1e3),
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(fp8.bf16_round(x), ref)


# ----------------------------------------------------------------------------
# quantisers
# ----------------------------------------------------------------------------
def _check_quant_bounds(x, deq, s_full):
    ax = np.abs(x)
    # normal e4m3 range: relative error <= 2^-4; subnormal range: absolute <= 2^-10 * s
    err = np.abs(deq - x)
    bound = np.maximum(ax * 2.0 ** -4, s_full * 2.0 ** -10) * (1 + 1e-6)
    assert np.all(err <= bound)


def test_quant_per_tensor_closed_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 256)).astype(np.float32) * 3
    q, s = spec.quant_per_tensor(x)
    assert s == np.float32(np.abs(x).max() / np.float32(448))
    i = np.unravel_index(np.abs(x).argmax(), x.shape)
    assert q[i] in (0x7E, 0xFE)
    _check_quant_bounds(x, spec.dequant_per_tensor(q, s), s)


def test_quant_group_and_block_closed_form():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((32, 384)).astype(np.float32)
    x[3, 128:256] = 0.0
    q, s = spec.quant_group_1x128(x)
    assert s.shape == (32, 3) and s[3, 1] == 1.0 and not q[3, 128:256].any()
    amax = np.abs(x.reshape(32, 3, 128)).max(2)
    np.testing.assert_array_equal(s[amax > 0], (amax / np.float32(448))[amax > 0])
    _check_quant_bounds(x, spec.dequant_group_1x128(q, s), np.repeat(s, 128, axis=1))
    w = rng.standard_normal((2, 256, 384)).astype(np.float32)
    qw, sw = spec.quant_block_128x128(w)
    assert sw.shape == (2, 2, 3)
    full = np.repeat(np.repeat(sw, 128, axis=1), 128, axis=2)
    _check_quant_bounds(w, spec.dequant_block_128x128(qw, sw), full)
    # the largest element of each block maps to +-448 exactly
    blocks = np.abs(w.reshape(2, 2, 128, 3, 128))
    for b in range(2):
        for i in range(2):
            for j in range(3):
                r, c = np.unravel_index(blocks[b, i, :, j, :].argmax(), (128, 128))
                assert qw[b, i * 128 + r, j * 128 + c] & 0x7F == 0x7E


def test_scale_floor_is_flt_min():
    x = np.zeros((1, 128), np.float32)
    x[0, 5] = np.float32(1e-40)
    q, s = spec.quant_group_1x128(x)
    assert s[0, 0] == np.float32(2.0 ** -126)


# ----------------------------------------------------------------------------
# routing
# ----------------------------------------------------------------------------
def test_route_topk_vs_torch_topk_softmax():
    rng = np.random.default_rng(4)
    for t, e, k in [(100, 8, 2), (64, 256, 8), (50, 128, 8), (33, 1024, 32)]:
        logits = rng.standard_normal((t, e)).astype(np.float32)
        idx, w = spec.route_topk(logits, k)
        tv, ti = torch.topk(torch.from_numpy(logits), k, dim=1, largest=True, sorted=True)
        np.testing.assert_array_equal(idx, ti.numpy())
        ref_w = torch.softmax(tv, dim=1).numpy()
        assert np.max(np.abs(w - ref_w) / ref_w) < 2e-6


def test_route_topk_ties_bruteforce_and_closed_form():
    rng = np.random.default_rng(5)
    logits = (np.round(rng.standard_normal((40, 12)) * 2) / 2).astype(np.float32)
    idx, w = spec.route_topk(logits, 5)
    for t in range(40):
        sel, ws = brute.topk_bruteforce(logits[t], 5)
        assert list(idx[t]) == sel
        np.testing.assert_allclose(w[t], ws, rtol=1e-6)
    idx, w = spec.route_topk(np.zeros((3, 10), np.float32), 4)
    np.testing.assert_array_equal(idx, np.tile(np.arange(4), (3, 1)))
    np.testing.assert_allclose(w, 0.25)


def test_counts_offsets_permutation_bruteforce():
    rng = np.random.default_rng(6)
    t, e, k = 23, 7, 3
    idx = np.stack([rng.choice(e, k, replace=False) for _ in range(t)]).astype(np.int32)
    counts, offsets = spec.expert_counts_offsets(idx, e)
    perm, inv = spec.permutation(idx, e)
    ref_counts = [sum(1 for tt in range(t) for j in range(k) if idx[tt, j] == x) for x in range(e)]
    assert list(counts) == ref_counts
    assert offsets[0] == 0 and offsets[-1] == t * k and list(np.diff(offsets)) == ref_counts
    ref_perm = [tt * k + j for x in range(e) for tt in range(t) for j in range(k) if idx[tt, j] == x]
    assert list(perm) == ref_perm
    assert list(inv[perm]) == list(range(t * k))


def test_permutation_invariants_full_size_dsv3():
    cfg = synth.CONFIGS["dsv3"]
    rng = np.random.default_rng(0)
    idx, _ = spec.route_topk(synth.make_logits(rng, cfg["T"], cfg["E"], cfg["skew"]), cfg["k"])
    counts, offsets = spec.expert_counts_offsets(idx, cfg["E"])
    perm, inv = spec.permutation(idx, cfg["E"])
    flat = idx.ravel()
    assert np.array_equal(np.sort(perm), np.arange(perm.size))
    assert np.all(np.diff(flat[perm]) >= 0)                          # expert-sorted
    for e in np.flatnonzero(counts)[:40]:
        seg = perm[offsets[e]:offsets[e + 1]]
        assert np.all(flat[seg] == e) and np.all(np.diff(seg) > 0)  # stable
    assert np.array_equal(inv[perm], np.arange(perm.size))
    assert (counts == 0).sum() > 0                                   # skew leaves experts empty


# ----------------------------------------------------------------------------
# GEMMs, epilogue, combine, whole layer
# ----------------------------------------------------------------------------
def test_gemm_pm1_known_answer():
    rng = np.random.default_rng(7)
    a = np.where(rng.integers(0, 2, (64, 256)) == 1, 0x38, 0xB8).astype(np.uint8)
    b = np.where(rng.integers(0, 2, (48, 256)) == 1, 0x38, 0xB8).astype(np.uint8)
    c = spec.gemm_fp8(a, b, np.float32(1), np.float32(1), out="f32")
    sa = np.where(a == 0x38, 1, -1).astype(np.int64)
    sb = np.where(b == 0x38, 1, -1).astype(np.int64)
    np.testing.assert_array_equal(c, (sa @ sb.T).astype(np.float32))


def test_gemm_vs_torch_matmul():
    d = synth.make_dense(96, 128, 256, seed=8)
    c = spec.gemm_fp8(d["a_q"], d["b_q"], d["sa"], d["sb"], out="f32")
    a = torch.from_numpy(d["a_q"]).view(torch.float8_e4m3fn).double() * float(d["sa"])
    b = torch.from_numpy(d["b_q"]).view(torch.float8_e4m3fn).double() * float(d["sb"])
    ref = (a @ b.T).numpy()
    assert np.max(np.abs(c - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_silu_mul_vs_torch():
    rng = np.random.default_rng(9)
    g = rng.standard_normal(4096).astype(np.float32) * 10
    u = rng.standard_normal(4096).astype(np.float32)
    ref = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    np.testing.assert_allclose(spec.silu_mul(g, u), ref, rtol=2e-6, atol=1e-30)


def test_combine_bruteforce():
    rng = np.random.default_rng(10)
    t, k, h = 9, 3, 16
    y = fp8.bf16_round(rng.standard_normal((t * k, h)).astype(np.float32))
    w = rng.random((t, k)).astype(np.float32)
    inv = rng.permutation(t * k).astype(np.int32)
    got = spec.combine(y, w, inv, rounded=False)
    for tt in range(t):
        acc = np.zeros(h, np.float32)
        for j in range(k):
            acc = (acc + w[tt, j] * y[inv[tt * k + j]]).astype(np.float32)
        np.testing.assert_array_equal(got[tt], acc)


@pytest.mark.parametrize("block,skew", [(False, False), (True, True)])
def test_moe_forward_vs_bruteforce(block, skew):
    d = synth.make_moe(T=24, H=256, I=128, E=8, k=3, block=block, skew=skew, seed=13)
    r = spec.moe_forward(d["x_q"], d["x_scale"], d["logits"], d["w13_q"], d["w13_s"], d["w2_q"],
                         d["w2_s"], d["k"], return_all=True)
    out, routes = brute.moe_bruteforce(d["x_q"], d["x_scale"], d["logits"], d["w13_q"], d["w13_s"],
                                       d["w2_q"], d["w2_s"], d["k"])
    for t, (sel, _) in enumerate(routes):
        assert list(r["topk_idx"][t]) == sel
    # both round h, y and out to bf16; summation-order differences move an
    # occasional element by one bf16 ulp (<= 2^-8 relative to the output max)
    assert spec.rel_err(r["out"], out) <= 2.0 ** -7


# ----------------------------------------------------------------------------
# golden fixtures (frozen oracle outputs)
# ----------------------------------------------------------------------------
def _golden_cases():
    return sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz")) if os.path.isdir(GOLDEN) else []


@pytest.mark.parametrize("name", _golden_cases())
def test_golden_fixture(name):
    g = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    if "mx_a" in g:
        for op, raw in (("a", "mx_a"), ("b", "mx_b")):
            q, s = mx.quant_mx(g[raw])
            np.testing.assert_array_equal(q, g[op + "_q"])
            np.testing.assert_array_equal(s, g["s" + op])
            np.testing.assert_array_equal(mx.mx_pack_scales(s), g["s" + op + "_packed"])
        np.testing.assert_array_equal(mx.gemm_mx(g["a_q"], g["sa"], g["b_q"], g["sb"]), g["c_f32"])
        return
    if "a_q" in g:
        c = spec.gemm_fp8(g["a_q"], g["b_q"], g["sa"], g["sb"], out="f32")
        np.testing.assert_array_equal(c, g["c_f32"])
        return
    xs = g["x_scale"] if g["x_scale"].ndim == 2 else np.float32(g["x_scale"])
    r = spec.moe_forward(g["x_q"], xs, g["logits"], g["w13_q"], g["w13_s"], g["w2_q"], g["w2_s"],
                         int(g["k"]), return_all=True)
    for key in ("topk_idx", "counts", "offsets", "perm", "inv_perm", "hq"):
        np.testing.assert_array_equal(r[key], g[key], err_msg=key)
    np.testing.assert_array_equal(r["topk_w"], g["topk_w"])
    np.testing.assert_array_equal(r["out"], g["out"])


def test_golden_fixtures_present():
    assert len(_golden_cases()) >= 3


# ----------------------------------------------------------------------------
# the pins have teeth: plausible mistakes planted in the oracle are caught
# ----------------------------------------------------------------------------
def test_planted_mistakes_are_caught(monkeypatch):
    rng = np.random.default_rng(11)
    logits = rng.standard_normal((30, 16)).astype(np.float32)
    tv, ti = torch.topk(torch.from_numpy(logits), 4, dim=1)
    # (1) ties broken toward the higher expert id disagree with the brute force
    ties = (np.round(rng.standard_normal((40, 12)) * 2) / 2).astype(np.float32)
    bad_idx = np.argsort(ties, axis=1, kind="stable")[:, ::-1][:, :5]
    ref_idx = np.array([brute.topk_bruteforce(ties[t], 5)[0] for t in range(40)])
    assert not np.array_equal(bad_idx, ref_idx)
    assert np.array_equal(spec.route_topk(ties, 5)[0], ref_idx)
    # (2) softmax over all experts instead of the selected ones
    bad_w = torch.softmax(torch.from_numpy(logits), 1).numpy()
    bad_w = np.take_along_axis(bad_w, ti.numpy(), 1)
    assert np.max(np.abs(bad_w - torch.softmax(tv, 1).numpy())) > 1e-3
    # (3) transposed weight operand in the GEMM fails the +-1 KAT
    a = np.where(rng.integers(0, 2, (32, 32)) == 1, 0x38, 0xB8).astype(np.uint8)
    b = np.where(rng.integers(0, 2, (32, 32)) == 1, 0x38, 0xB8).astype(np.uint8)
    good = spec.gemm_fp8(a, b, np.float32(1), np.float32(1), out="f32")
    monkeypatch.setattr(spec, "dequant_per_tensor", lambda q, s: fp8.e4m3_to_f32(q).T * np.float32(s))
    bad = spec.gemm_fp8(a, b, np.float32(1), np.float32(1), out="f32")
    assert not np.array_equal(good, bad)
    monkeypatch.undo()
    # (4) a dropped scale (block scale ignored) breaks the layer-level brute-force pin
    d = synth.make_moe(T=12, H=256, I=128, E=4, k=2, block=True, skew=False, seed=14)
    out_ref, _ = brute.moe_bruteforce(d["x_q"], d["x_scale"], d["logits"], d["w13_q"], d["w13_s"],
                                      d["w2_q"], d["w2_s"], d["k"])
    monkeypatch.setattr(spec, "dequant_group_1x128", lambda q, s: fp8.e4m3_to_f32(q))
    bad_out = spec.moe_forward(d["x_q"], d["x_scale"], d["logits"], d["w13_q"], d["w13_s"], d["w2_q"],
                               d["w2_s"], d["k"])
    assert spec.rel_err(bad_out, out_ref) > 1e-2
