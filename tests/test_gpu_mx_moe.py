"""MX (1x32 e8m0) MoE layer through the native path vs the oracle (oracle/mx.py).

Bars, stage by stage on identical inputs: routing, offsets and permutation
bit-exact (the shared kernels); the exponent word layouts bit-exact; h within
1e-2 relative error of the oracle's fp32 value; GEMM 1's fused MX
requantisation bit-exact against quant_mx of the GPU's own bf16 h; y (from the
GPU's hq) and the combine (from the GPU's y) within 1e-2 of the fp32 values;
the one-call layer, the stepwise layer and packed vs row-major weights give
identical bits.

End to end against an independent oracle run, at config 3's shapes (I = 2048)
the sampled tokens meet TOL (2.8e-3 measured).  The small shapes below (I of
128-384) are held to E2E_TOL = 3e-2: the MX requantisation of h rounds to
3-bit mantissas under power-of-two block scales, so a one-ulp bf16 difference
in h (fp32 accumulation order) can move an element of hq by a whole e4m3 step
(up to 6.25%), and with few terms per output one such step weighs more (1.0e-3
to 1.03e-2 measured over three seeds of each case).
"""
import numpy as np
import pytest
import torch

from helpers import bf16_np, f8_np, rel_err, to_f8, to_f32
from oracle import fp8, mx, spec

pytestmark = pytest.mark.gpu
TOL = 1e-2
E2E_TOL = 3e-2

CASES = {
    "e8k3_skew": dict(T=40, H=256, I=128, E=8, k=3, skew=True),
    "e64k8_skew": dict(T=300, H=768, I=384, E=64, k=8, skew=True),
    "e12k8": dict(T=8, H=256, I=256, E=12, k=8, skew=False),
}


def _u8(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).cuda()


def _inputs(name, seed=31):
    d = mx.make_mx_moe(seed=seed, **CASES[name])
    g = dict(x_q=to_f8(d["x_q"]), x_e8m0=_u8(d["x_e8m0"]), logits=to_f32(d["logits"]),
             w13_q=to_f8(d["w13_q"]), w13_e8m0=_u8(d["w13_e8m0"]), w2_q=to_f8(d["w2_q"]),
             w2_e8m0=_u8(d["w2_e8m0"]), k=d["k"])
    return d, g


def _words(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("gate_up", [False, True])
def test_pack_weight_words_bit_exact(hk, gate_up):
    rng = np.random.default_rng(4 + gate_up)
    s = rng.integers(0, 255, (5, 512, 768 // 32), dtype=np.uint8)
    w = hk.mx_pack_weight_scales(_u8(s), gate_up=gate_up)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_words(w), mx.pack_weight_words(s, gate_up=256 if gate_up else 0))


@pytest.mark.parametrize("name", list(CASES))
def test_mx_layer_stepwise(hk, name):
    d, g = _inputs(name)
    ref = mx.moe_forward_mx(d["x_q"], d["x_e8m0"], d["logits"], d["w13_q"], d["w13_e8m0"], d["w2_q"],
                            d["w2_e8m0"], d["k"], return_all=True)
    w13w = hk.mx_pack_weight_scales(g["w13_e8m0"], gate_up=True)
    w2w = hk.mx_pack_weight_scales(g["w2_e8m0"])
    r = hk.moe_forward_mx_steps(g["x_q"], g["x_e8m0"], g["logits"], g["w13_q"], w13w, g["w2_q"], w2w,
                                g["k"], keep_h=True)
    torch.cuda.synchronize()
    # shared routing kernels: bit-exact
    np.testing.assert_array_equal(r["offsets"].cpu().numpy(), ref["offsets"])
    np.testing.assert_array_equal(r["perm"].cpu().numpy(), ref["perm"])
    rows, e = int(ref["offsets"][-1]), CASES[name]["E"]
    ws = mx.tile_words_per_step(rows, e)
    # gathered activation words (written for the M tiles that exist; the rest of
    # the ws words per step are never read)
    n_mt = int(r["mtile_offsets"].cpu().numpy()[-1])
    used = slice(0, n_mt * 256)
    np.testing.assert_array_equal(_words(r["xw"])[:, used], mx.gather_words(ref["xs"], ref["offsets"], e)[:, used])
    # GEMM 1's h against the oracle's fp32 value, and the fused requantisation
    # against quant_mx of the GPU's own bf16 h (bit-exact, words included)
    h_gpu = bf16_np(r["h"])
    assert rel_err(h_gpu, ref["h"]) <= TOL
    hq_ref, hs_ref = mx.quant_mx(h_gpu)
    np.testing.assert_array_equal(f8_np(r["hq"]), hq_ref)
    hw = _words(r["hw"])
    assert hw.shape == (CASES[name]["I"] // 128, ws)
    np.testing.assert_array_equal(hw[:, used], mx.gather_words(hs_ref, ref["offsets"], e)[:, used])
    # GEMM 2 from the GPU's own hq: within tolerance of the fp32 product
    offs = ref["offsets"]
    y_ref = np.zeros((rows, CASES[name]["H"]), np.float32)
    for ex in range(e):
        lo, hi = int(offs[ex]), int(offs[ex + 1])
        if hi > lo:
            y_ref[lo:hi] = mx.dequant_mx(hq_ref[lo:hi], hs_ref[lo:hi]) @ mx.dequant_mx(d["w2_q"][ex], d["w2_e8m0"][ex]).T
    y_gpu = bf16_np(r["y"])
    assert rel_err(y_gpu, y_ref) <= TOL
    # combine from the GPU's own y, then the whole layer end to end
    comb = spec.combine(y_gpu, r["topk_w"].cpu().numpy(), r["inv_perm"].cpu().numpy(), rounded=False)
    assert rel_err(bf16_np(r["out"]), comb) <= TOL
    assert rel_err(bf16_np(r["out"]), ref["out_f32"]) <= E2E_TOL


@pytest.mark.parametrize("name", ["e8k3_skew", "e64k8_skew"])
def test_mx_layer_one_call_packed_and_rows(hk, name):
    """MoELayerMX (one C call, packed weights) == the stepwise layer with
    row-major weights, bit for bit, also on a reused workspace."""
    d, g = _inputs(name, seed=33)
    w13w = hk.mx_pack_weight_scales(g["w13_e8m0"], gate_up=True)
    w2w = hk.mx_pack_weight_scales(g["w2_e8m0"])
    steps = hk.moe_forward_mx_steps(g["x_q"], g["x_e8m0"], g["logits"], g["w13_q"], w13w, g["w2_q"], w2w,
                                    g["k"], packed=False)
    layer = hk.MoELayerMX(g["w13_q"], g["w13_e8m0"], g["w2_q"], g["w2_e8m0"], g["k"])
    out1 = layer(g["x_q"], g["x_e8m0"], g["logits"])
    out2 = layer(g["x_q"], g["x_e8m0"], g["logits"])  # dirty workspace
    torch.cuda.synchronize()
    assert torch.equal(out1.view(torch.int16), steps["out"].view(torch.int16))
    assert torch.equal(out2.view(torch.int16), out1.view(torch.int16))
    ref = mx.moe_forward_mx(d["x_q"], d["x_e8m0"], d["logits"], d["w13_q"], d["w13_e8m0"], d["w2_q"],
                            d["w2_e8m0"], d["k"], return_all=True)
    assert rel_err(bf16_np(out1), ref["out_f32"]) <= E2E_TOL


def test_mx_layer_dsv3_shape_sampled(hk):
    """Config-3 shapes (T=8192, H=7168, I=2048, E=256, top-8, Zipf skew) in MX
    format: bit-identical one-call vs stepwise, and sampled tokens vs the
    oracle's per-token computation."""
    T, H, I, E, k = 8192, 7168, 2048, 256, 8
    gen = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn((T, H), generator=gen, device="cuda")
    x_q, x_e = hk.quant_mx(x)
    del x
    logits = torch.randn((T, E), generator=gen, device="cuda")
    rank = torch.randperm(E, generator=gen, device="cuda").float() + 1.0
    logits += (-1.1 * torch.log(rank))[None, :]
    w13_q = torch.empty((E, 2 * I, H), dtype=torch.float8_e4m3fn, device="cuda")
    w13_e = torch.empty((E, 2 * I, H // 32), dtype=torch.uint8, device="cuda")
    w2_q = torch.empty((E, H, I), dtype=torch.float8_e4m3fn, device="cuda")
    w2_e = torch.empty((E, H, I // 32), dtype=torch.uint8, device="cuda")
    for e0 in range(0, E, 16):
        w = torch.randn((16 * 2 * I, H), generator=gen, device="cuda")
        q, s = hk.quant_mx(w)
        w13_q[e0:e0 + 16].copy_(q.view(16, 2 * I, H))
        w13_e[e0:e0 + 16].copy_(s.view(16, 2 * I, H // 32))
        w = torch.randn((16 * H, I), generator=gen, device="cuda")
        q, s = hk.quant_mx(w)
        w2_q[e0:e0 + 16].copy_(q.view(16, H, I))
        w2_e[e0:e0 + 16].copy_(s.view(16, H, I // 32))
    del w, q, s
    layer = hk.MoELayerMX(w13_q, w13_e, w2_q, w2_e, k)
    out = layer(x_q, x_e, logits)
    w13w = hk.mx_pack_weight_scales(w13_e, gate_up=True)
    w2w = hk.mx_pack_weight_scales(w2_e)
    steps = hk.moe_forward_mx_steps(x_q, x_e, logits, w13_q, w13w, w2_q, w2w, k)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), steps["out"].view(torch.int16))
    counts = steps["counts"].cpu().numpy()
    assert (counts == 0).sum() > 0  # skewed: some experts get no tokens
    # sampled tokens, per-token oracle (routing from the GPU's bit-exact top-k)
    idx = steps["topk_idx"].cpu().numpy()
    wts = steps["topk_w"].cpu().numpy()
    toks = np.random.default_rng(2).choice(T, 6, replace=False)
    xq, xe = f8_np(x_q[torch.from_numpy(toks).cuda()]), x_e[torch.from_numpy(toks).cuda()].cpu().numpy()
    ref = np.zeros((len(toks), H), np.float32)
    for n, t in enumerate(toks):
        xt = mx.dequant_mx(xq[n:n + 1], xe[n:n + 1])
        acc = np.zeros(H, np.float32)
        for j in range(k):
            e = int(idx[t, j])
            z = (xt @ mx.dequant_mx(f8_np(w13_q[e]), w13_e[e].cpu().numpy()).T).astype(np.float32)
            h = fp8.bf16_round(spec.silu_mul(z[:, :I], z[:, I:]))
            hq, hs = mx.quant_mx(h)
            y = (mx.dequant_mx(hq, hs) @ mx.dequant_mx(f8_np(w2_q[e]), w2_e[e].cpu().numpy()).T)
            acc += wts[t, j] * fp8.bf16_round(y.astype(np.float32))[0]
        ref[n] = acc
    got = bf16_np(out[torch.from_numpy(toks).cuda()])
    assert rel_err(got, ref) <= TOL
