"""MoE path through the native kernels vs the oracle (same seeded inputs).

Bars (from the path's specification):
  * bit-exact: top-k indices, counts, offsets, M-tile offsets, perm, inv_perm,
    the gathered expert-contiguous rows and scales, requantised bytes/scales
    (fed the GPU's own bf16 intermediate), device quantisers;
  * routing weights: max relative error <= 1e-6 (fp32 exp/divide);
  * GEMM and combine outputs: max|got - ref| / max|ref| <= 1e-2, ref = the
    fp32 value before the bf16 store.
"""
import numpy as np
import pytest
import torch

from helpers import bf16_np, f8_np, moe_inputs_to_gpu, rel_err, to_f32, to_f8
from oracle import spec, synth

pytestmark = pytest.mark.gpu
TOL = 1e-2

SMALL = {
    "tensor_e8k2": dict(T=96, H=512, I=256, E=8, k=2, block=False, skew=False),
    "block_e16k4_skew": dict(T=130, H=512, I=256, E=16, k=4, block=True, skew=True),
    "block_e64k8_skew": dict(T=300, H=768, I=384, E=64, k=8, block=True, skew=True),
    "tensor_e5k5": dict(T=33, H=256, I=128, E=5, k=5, block=False, skew=False),
    "block_t1": dict(T=1, H=256, I=128, E=4, k=2, block=True, skew=False),
}


def _np(t):
    return t.detach().cpu().numpy()


def _run_steps(hk, g, keep_h=True):
    r = hk.moe_forward_steps(g["x_q"], g["x_scale"], g["logits"], g["w13_q"], g["w13_scale"],
                             g["w2_q"], g["w2_scale"], g["top_k"], keep_h=keep_h)
    torch.cuda.synchronize()
    return r


@pytest.mark.parametrize("name", list(SMALL))
def test_moe_stepwise_parity(hk, name):
    d = synth.make_moe(seed=11, **SMALL[name])
    g = moe_inputs_to_gpu(d)
    r = _run_steps(hk, g)
    ref = spec.moe_forward(d["x_q"], d["x_scale"], d["logits"], d["w13_q"], d["w13_s"], d["w2_q"],
                           d["w2_s"], d["k"], return_all=True)
    block = SMALL[name]["block"]
    # routing: bit-exact
    np.testing.assert_array_equal(_np(r["topk_idx"]), ref["topk_idx"])
    assert rel_err(_np(r["topk_w"]), ref["topk_w"]) <= 1e-6
    np.testing.assert_array_equal(_np(r["counts"]), ref["counts"])
    np.testing.assert_array_equal(_np(r["offsets"]), ref["offsets"])
    mt = np.concatenate([[0], np.cumsum((ref["counts"] + 255) // 256)])
    np.testing.assert_array_equal(_np(r["mtile_offsets"]), mt)
    np.testing.assert_array_equal(_np(r["perm"]), ref["perm"])
    np.testing.assert_array_equal(_np(r["inv_perm"]), ref["inv_perm"])
    # GEMM1 + SiLU*up (token rows gathered through perm): tolerance vs fp32
    h = bf16_np(r["h"])
    h_ref32 = spec.gemm1_silu(ref["xp"], ref["xps"], d["w13_q"], d["w13_s"], ref["offsets"], rounded=False)
    assert rel_err(h, h_ref32) <= TOL
    # requantisation of the GPU's own bf16 h: bit-exact (block mode: fused into
    # GEMM 1's epilogue; per-tensor mode: the requant kernel)
    hq_ref, hs_ref = spec.requant(h, block)
    np.testing.assert_array_equal(f8_np(r["hq"]), hq_ref)
    if block:
        np.testing.assert_array_equal(_np(r["hs"]).T, hs_ref)
    else:
        assert _np(r["hs"])[0] == hs_ref
    # GEMM2 from the GPU's own hq
    y_ref32 = spec.gemm2(hq_ref, hs_ref, d["w2_q"], d["w2_s"], ref["offsets"], rounded=False)
    assert rel_err(bf16_np(r["y"]), y_ref32) <= TOL
    # combine from the GPU's own y
    out_ref32 = spec.combine(bf16_np(r["y"]), _np(r["topk_w"]), ref["inv_perm"], rounded=False)
    assert rel_err(bf16_np(r["out"]), out_ref32) <= TOL
    # end to end against the oracle's own pipeline
    assert rel_err(bf16_np(r["out"]), ref["out_f32"]) <= TOL


@pytest.mark.parametrize("block", [False, True])
def test_scatter_row_copy(hk, block):
    """hkmoe_scatter with x_q: the permuted row copy (and transposed scales) is bit-exact."""
    d = synth.make_moe(T=70, H=512, I=128, E=12, k=3, block=block, skew=True, seed=4)
    g = moe_inputs_to_gpu(d)
    ref = spec.moe_forward(d["x_q"], d["x_scale"], d["logits"], d["w13_q"], d["w13_s"], d["w2_q"],
                           d["w2_s"], d["k"], return_all=True)
    t, k, e, hdim = 70, 3, 12, 512
    r = _run_steps(hk, g, keep_h=False)
    perm = torch.empty_like(r["perm"])
    inv = torch.empty_like(r["inv_perm"])
    xp = torch.empty((t * k, hdim), dtype=torch.float8_e4m3fn, device="cuda")
    xps = torch.empty((hdim // 128, t * k), dtype=torch.float32, device="cuda") if block else None
    hk.tk_kernel.dispatch_scatter(r["topk_idx"], r["offsets"], r["block_base"], perm, inv, g["x_q"],
                                  g["x_scale"] if block else None, xp, xps)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_np(perm), ref["perm"])
    np.testing.assert_array_equal(f8_np(xp), ref["xp"])
    if block:
        np.testing.assert_array_equal(_np(xps).T, ref["xps"])
    del e


@pytest.mark.parametrize("name", ["tensor_e8k2", "block_e16k4_skew"])
def test_moe_single_call_matches_steps(hk, name):
    """hkmoe_moe_forward (one C call, carved workspace) == the stepwise path, bit for bit."""
    d = synth.make_moe(seed=12, **SMALL[name])
    g = moe_inputs_to_gpu(d)
    r = _run_steps(hk, g, keep_h=False)
    out = hk.moe_forward(g["x_q"], g["x_scale"], g["logits"], g["w13_q"], g["w13_scale"],
                         g["w2_q"], g["w2_scale"], g["top_k"])
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), r["out"].view(torch.int16))
    # second call with a reused (dirty) workspace gives the same bits
    layer = hk.MoELayer(g["w13_q"], g["w13_scale"], g["w2_q"], g["w2_scale"], g["top_k"])
    o1 = layer(g["x_q"], g["x_scale"], g["logits"]).clone()
    o2 = layer(g["x_q"], g["x_scale"], g["logits"])
    torch.cuda.synchronize()
    assert torch.equal(o1.view(torch.int16), o2.view(torch.int16))
    assert torch.equal(o1.view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("t,e,k,block", [(1, 8, 2, True), (33, 16, 4, False), (512, 64, 8, True),
                                         (513, 64, 8, True), (200, 1024, 32, True), (96, 300, 7, False)])
def test_layer_small_batches_match_steps(hk, t, e, k, block):
    """The one-call layer (narrow schedule, block scan inside expert_offsets up
    to 16 routing blocks) against the stepwise path (separate kernels, 256x256
    GEMMs only), bit for bit: T = 1, 33, 512 (16 routing blocks) and 513, E =
    1024 (64 experts per lane of a token's top-k row), k = 32, E not a power
    of two, with and without block scales."""
    print(f"one-call vs stepwise T={t} E={e} k={k} block={block}", flush=True)
    # inputs drawn and quantised on the device (E = 1024 weights are slow to
    # make on the host); both paths see the same tensors
    gen = torch.Generator(device="cuda").manual_seed(21)
    x = torch.randn((t, 256), device="cuda", generator=gen)
    logits = torch.randn((t, e), device="cuda", generator=gen)
    logits -= 1.1 * torch.log1p(torch.randperm(e, device="cuda", generator=gen).float())  # skewed routing
    w13 = torch.randn((e, 256, 256), device="cuda", generator=gen)
    w2 = torch.randn((e, 256, 128), device="cuda", generator=gen)
    if block:
        x_q, x_s = hk.quant_group(x)
        w13_q, w13_s = hk.quant_block(w13)
        w2_q, w2_s = hk.quant_block(w2)
    else:
        x_q, x_s = hk.quant_tensor(x)
        w13_q, s13 = hk.quant_tensor(w13.reshape(e * 256, 256))
        w2_q, s2 = hk.quant_tensor(w2.reshape(e * 256, 128))
        w13_q, w2_q = w13_q.view(e, 256, 256), w2_q.view(e, 256, 128)
        w13_s, w2_s = s13.expand(e).contiguous(), s2.expand(e).contiguous()
    g = dict(x_q=x_q, x_scale=x_s, logits=logits, w13_q=w13_q, w13_scale=w13_s, w2_q=w2_q, w2_scale=w2_s,
             top_k=k)
    r = _run_steps(hk, g, keep_h=False)
    out = hk.moe_forward(g["x_q"], g["x_scale"], g["logits"], g["w13_q"], g["w13_scale"],
                         g["w2_q"], g["w2_scale"], g["top_k"])
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), r["out"].view(torch.int16))


def test_layer_concurrent_host_threads(hk):
    """Two host threads, each with its own layer and its own (default-priority)
    stream, run the two-stream layer at the same time: their narrow kernels share
    the library's auxiliary stream and fork/join events, which a lock held over
    each call's launch sequence keeps apart.  Every output equals the serial
    result bit for bit."""
    import threading
    t, e, k = 1536, 64, 8  # T*k = 12288 > 2*E*64 rows: narrow experts beside 256x256 ones, two streams
    gen = torch.Generator(device="cuda").manual_seed(5)
    w13_q, w13_s = hk.quant_block(torch.randn((e, 512, 512), device="cuda", generator=gen))
    w2_q, w2_s = hk.quant_block(torch.randn((e, 512, 256), device="cuda", generator=gen))
    batches = []
    for _ in range(2):
        x_q, x_s = hk.quant_group(torch.randn((t, 512), device="cuda", generator=gen))
        logits = torch.randn((t, e), device="cuda", generator=gen)
        logits -= 1.1 * torch.log1p(torch.randperm(e, device="cuda", generator=gen).float())
        counts = torch.bincount(torch.topk(logits, k, dim=1).indices.flatten(), minlength=e)
        assert int(((counts > 0) & (counts <= 64)).sum()) > 0 and int((counts > 256).sum()) > 0
        batches.append((x_q, x_s, logits))
    layers = [hk.MoELayer(w13_q, w13_s, w2_q, w2_s, k) for _ in range(2)]
    refs = [layers[i](*batches[i]).clone() for i in range(2)]
    torch.cuda.synchronize()
    outs, errors = [[], []], []

    def run(i):
        s = torch.cuda.Stream()
        try:
            with torch.cuda.stream(s):
                for _ in range(6):
                    outs[i].append(layers[i](*batches[i]).clone())
            s.synchronize()
        except Exception as ex:  # reported below, in the test's thread
            errors.append(ex)

    print(f"concurrent layers T={t} E={e} k={k}, two host threads", flush=True)
    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a layer thread did not finish"
    assert not errors, errors
    for i in range(2):
        assert len(outs[i]) == 6
        for o in outs[i]:
            assert torch.equal(o.view(torch.int16), refs[i].view(torch.int16))


@pytest.mark.parametrize("name", ["tensor_e8k2", "block_e16k4_skew"])
def test_moe_empty_batch(hk, name):
    """T = 0 tokens: the layer returns an empty [0, H] output and launches nothing
    that fails; the same layer then still matches the stepwise path."""
    d = synth.make_moe(seed=13, **SMALL[name])
    g = moe_inputs_to_gpu(d)
    layer = hk.MoELayer(g["w13_q"], g["w13_scale"], g["w2_q"], g["w2_scale"], g["top_k"])
    hdim = g["x_q"].shape[1]
    x0 = g["x_q"][:0]
    s0 = g["x_scale"][:, :0] if g["x_scale"].dim() == 2 else g["x_scale"]
    out0 = layer(x0, s0, g["logits"][:0])
    torch.cuda.synchronize()
    assert tuple(out0.shape) == (0, hdim) and out0.dtype == torch.bfloat16
    out = layer(g["x_q"], g["x_scale"], g["logits"])
    r = _run_steps(hk, g, keep_h=False)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), r["out"].view(torch.int16))
    out0 = layer(x0, s0, g["logits"][:0])
    torch.cuda.synchronize()
    assert tuple(out0.shape) == (0, hdim)
    # the stepwise path (routing, scatter, both grouped GEMMs, combine) on no rows
    r0 = hk.moe_forward_steps(x0, s0, g["logits"][:0], g["w13_q"], g["w13_scale"], g["w2_q"],
                              g["w2_scale"], g["top_k"])
    torch.cuda.synchronize()
    assert tuple(r0["out"].shape) == (0, hdim)


def test_empty_dense_and_quantisers(hk):
    """M = 0 / no rows: the dense GEMMs and the quantisers return empty results."""
    a = torch.empty((0, 256), dtype=torch.float32, device="cuda")
    b = torch.randn((256, 256), device="cuda")
    aq, sa = hk.quant_tensor(a)
    bq, sb = hk.quant_tensor(b)
    c = hk.gemm_fp8(aq, bq, sa, sb)
    gq, gs = hk.quant_group(a)
    mq, ms = hk.quant_mx(a)
    bmq, bms = hk.quant_mx(b)
    cm = hk.gemm_mx(mq, hk.mx_pack_scales(ms), bmq, hk.mx_pack_scales(bms))
    torch.cuda.synchronize()
    assert tuple(c.shape) == (0, 256) and tuple(cm.shape) == (0, 256)
    assert aq.numel() == 0 and gq.numel() == 0 and mq.numel() == 0 and gs.numel() == 0
    assert torch.isfinite(sa).all()


@pytest.mark.parametrize("name", ["tensor_e8k2", "block_e16k4_skew", "block_e64k8_skew", "tensor_e5k5"])
def test_packed_weights_bit_exact(hk, name):
    """Grouped GEMMs on hkmoe_pack_weights output == on row-major weights, bit
    for bit, in every intermediate (the pack is a pure relayout)."""
    d = synth.make_moe(seed=13, **SMALL[name])
    g = moe_inputs_to_gpu(d)
    w13p = hk.pack_weights(g["w13_q"], gate_up=True)
    w2p = hk.pack_weights(g["w2_q"])
    torch.cuda.synchronize()
    # a relayout: the same multiset of bytes, and not the identity
    for w, p in ((g["w13_q"], w13p), (g["w2_q"], w2p)):
        wb, pb = w.view(torch.uint8).flatten(), p.view(torch.uint8).flatten()
        assert torch.equal(torch.sort(wb).values, torch.sort(pb).values)
        assert not torch.equal(wb, pb)
    ref = _run_steps(hk, g, keep_h=True)
    r = hk.moe_forward_steps(g["x_q"], g["x_scale"], g["logits"], w13p, g["w13_scale"], w2p,
                             g["w2_scale"], g["top_k"], keep_h=True, packed=True)
    torch.cuda.synchronize()
    for key in ("h", "hq", "hs", "y", "out"):
        a, b = ref[key], r[key]
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), key
    out = hk.moe_forward(g["x_q"], g["x_scale"], g["logits"], w13p, g["w13_scale"], w2p,
                         g["w2_scale"], g["top_k"], packed=True)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref["out"].view(torch.int16))


@pytest.mark.parametrize("name", ["block_e64k8_skew", "tensor_e8k2"])
def test_mtile_list_order_and_results(hk, name):
    """The M-tile list holds every (expert, first row) tile exactly once: the
    experts with at least one full 256-row tile first, each with all its tiles
    in row order (expert order), then the single partial tiles of the smaller
    experts; the grouped GEMMs give the same bits with and without it (it only
    orders the tiles)."""
    d = synth.make_moe(seed=21, **SMALL[name])
    g = moe_inputs_to_gpu(d)
    r = _run_steps(hk, g, keep_h=False)   # uses the list
    counts, offs = _np(r["counts"]), _np(r["offsets"])
    n_mt = int(_np(r["mtile_offsets"])[-1])
    lst = _np(r["mtile_list"])[:2 * n_mt].reshape(n_mt, 2)
    head = [(e, offs[e] + 256 * s) for e in range(len(counts)) if counts[e] >= 256
            for s in range((counts[e] + 255) // 256)]
    tail = [(e, offs[e]) for e in range(len(counts)) if 0 < counts[e] < 256]
    assert [tuple(x) for x in lst] == head + tail
    assert any(counts[e] >= 256 and counts[e] % 256 for e in range(len(counts))) or name != "block_e64k8_skew"
    # the same layer without the list (expert order): identical intermediates
    e = len(counts)
    tc = torch.zeros(16, dtype=torch.int32, device="cuda")
    block = SMALL[name]["block"]
    hq2, hs2 = torch.empty_like(r["hq"]), torch.empty_like(r["hs"])
    if block:
        hk.tk_kernel.dispatch_grouped_gemm1(g["x_q"], g["x_scale"], r["perm"], g["top_k"], g["w13_q"],
                                            g["w13_scale"], r["offsets"], r["mtile_offsets"], hq2, hs2, tc[:8])
    else:
        h2, amax2 = torch.empty_like(r["h"]), torch.zeros(1, dtype=torch.float32, device="cuda")
        hk.tk_kernel.dispatch_grouped_gemm1(g["x_q"], g["x_scale"], r["perm"], g["top_k"], g["w13_q"],
                                            g["w13_scale"], r["offsets"], r["mtile_offsets"], h2, amax2, tc[:8])
        hk.tk_kernel.dispatch_requant(h2, amax2, hq2, hs2)
    y2 = torch.empty_like(r["y"])
    hk.tk_kernel.dispatch_grouped_gemm2(hq2, hs2, g["w2_q"], g["w2_scale"], r["offsets"], r["mtile_offsets"],
                                        y2, tc[8:])
    torch.cuda.synchronize()
    assert torch.equal(hq2.view(torch.uint8), r["hq"].view(torch.uint8))
    assert torch.equal(hs2, r["hs"])
    assert torch.equal(y2.view(torch.int16), r["y"].view(torch.int16))
    del e


def _quotient_check_cases():
    """The number of (x, s) pairs hkmoe_requant_quotient_check enumerates."""
    n = 0
    for y in range(37):  # normal x: ea = -126 + 7y, g = 0 .. 40 with x >= 2^-126, x <= amax
        ea = -126 + 7 * y
        for ma in range(128):
            for g in range(41):
                if ea - g < -126:
                    break
                n += 2 * (ma + 1 if g == 0 else 128)
    n += 27 * 128 * 128 * 2  # bf16 subnormals and zeros x = +-mx 2^-133, amax exponents -126 .. -100
    n += 127 * 128 * 2 + 2  # amax = inf: finite x, and x = +-inf
    return n


def test_requant_quotient_matches_division(hk):
    """The GEMM 1 epilogues divide each value by its group scale as a product
    with the correctly rounded reciprocal plus one exact-remainder FMA step.
    That must give the IEEE quotient bit for bit (the requantisation is
    bit-exact against the oracle): checked on the device over every bf16 value
    against every bf16 row maximum, exponents sampled across the range."""
    counts = torch.zeros(2, dtype=torch.int32, device="cuda")
    hk.tk_kernel.dispatch_requant_quotient_check(counts)
    torch.cuda.synchronize()
    cases, bad = (int(v) for v in counts.cpu())
    assert cases == _quotient_check_cases()
    assert bad == 0, f"{bad} of {cases} quotients differ from x / s"


@pytest.mark.parametrize("block", [True, False])
def test_requant_large_bit_exact(hk, block):
    """Requantisation of 8M bf16 values (log-normal row magnitudes, plus rows
    whose values sit on and next to e4m3 rounding midpoints) is bit-exact
    against the oracle (the quotient x / s correctly rounded, then RNE to
    e4m3, including the ties at midpoints)."""
    rng = np.random.default_rng(31)
    rows, inter = 4096, 2048
    h = rng.standard_normal((rows, inter)).astype(np.float32)
    h *= np.exp(rng.standard_normal((rows, 1)) * 3).astype(np.float32)
    # row 0: amax 448 (scale exactly 1): every e4m3 midpoint and its bf16 neighbours
    codes = np.arange(1, 0x7E, dtype=np.uint8)
    v = spec.dequant_per_tensor(codes, np.float32(1.0)).astype(np.float32)
    mid = ((v[:-1] + v[1:]) / 2).astype(np.float32)
    near = np.concatenate([mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1e9))])
    near = spec.bf16_round(near)
    row = np.resize(np.concatenate([near, -near]), inter).astype(np.float32)
    row[0] = 448.0
    h[0] = row
    h = spec.bf16_round(h)
    hb = torch.from_numpy(h).to(torch.bfloat16).cuda()
    hq = torch.empty((rows, inter), dtype=torch.float8_e4m3fn, device="cuda")
    if block:
        hs = torch.empty((inter // 128, rows), dtype=torch.float32, device="cuda")
        hk.tk_kernel.dispatch_requant(hb, None, hq, hs)
    else:
        hs = torch.empty(1, dtype=torch.float32, device="cuda")
        amax = torch.tensor([float(np.abs(h).max())], dtype=torch.float32, device="cuda")
        hk.tk_kernel.dispatch_requant(hb, amax, hq, hs)
    torch.cuda.synchronize()
    q_ref, s_ref = spec.requant(h, block)
    np.testing.assert_array_equal(f8_np(hq), q_ref)
    if block:
        np.testing.assert_array_equal(_np(hs).T, s_ref)
    else:
        assert _np(hs)[0] == s_ref


@pytest.mark.parametrize("case", ["finite", "inf", "nan"])
def test_requant_tensor_special_values(hk, case):
    """Per-tensor requantisation with infinities and NaNs in h, against the
    specification's bytes: an infinite h makes amax and s infinite (finite x
    give signed zeros); a NaN makes amax NaN and s = 1, so an infinite x
    saturates to +-448.  Signed zeros and values next to the saturation point
    ride along.  Where the specification's quotient is NaN (a NaN x, or
    inf / inf) the device conversion's clamp gives +-448 (0x7E | sign), not the
    NaN code 0x7F, as documented for non-finite inputs."""
    rng = np.random.default_rng(5)
    rows, inter = 64, 2048
    h = (rng.standard_normal((rows, inter)) * 40).astype(np.float32)
    h[0, :8] = [0.0, -0.0, 448.0, -448.0, 464.0, -464.0, 465.0, 1e-30]
    if case in ("inf", "nan"):
        h[1, :4] = [np.inf, -np.inf, np.inf, -np.inf]
    if case == "nan":
        h[2, :2] = [np.nan, -np.nan]
    h = spec.bf16_round(h)
    hb = torch.from_numpy(h).to(torch.bfloat16).cuda()
    hq = torch.empty((rows, inter), dtype=torch.float8_e4m3fn, device="cuda")
    hs = torch.empty(1, dtype=torch.float32, device="cuda")
    amax = torch.tensor([float(np.max(np.abs(h)))], dtype=torch.float32, device="cuda")
    hk.tk_kernel.dispatch_requant(hb, amax, hq, hs)
    torch.cuda.synchronize()
    with np.errstate(invalid="ignore"):
        q_ref, s_ref = spec.requant(h, False)
    got = f8_np(hq)
    nan = (q_ref & 0x7F) == 0x7F
    assert nan.sum() == {"finite": 0, "inf": 4, "nan": 2}[case]
    np.testing.assert_array_equal(got[~nan], q_ref[~nan])
    np.testing.assert_array_equal(got[nan] & 0x7F, np.full(int(nan.sum()), 0x7E, np.uint8))
    assert _np(hs)[0] == s_ref


def test_routing_ties_and_edges(hk):
    """Ties resolve to the lower expert id; T not a multiple of the block; E not a power of 2."""
    rng = np.random.default_rng(3)
    for t, e, k in [(1, 1, 1), (45, 100, 7), (70, 256, 8), (33, 1024, 32), (64, 3, 3)]:
        logits = np.round(rng.standard_normal((t, e)).astype(np.float32) * 2) / 2  # many ties
        idx_ref, w_ref = spec.route_topk(logits, k)
        lg = to_f32(logits)
        nblk = hk.tk_kernel.route_blocks(t)
        idx = torch.empty((t, k), dtype=torch.int32, device="cuda")
        w = torch.empty((t, k), dtype=torch.float32, device="cuda")
        bc = torch.empty((nblk, e), dtype=torch.int32, device="cuda")
        hk.tk_kernel.dispatch_route_topk(lg, idx, w, bc)
        counts = torch.empty(e, dtype=torch.int32, device="cuda")
        offs = torch.empty(e + 1, dtype=torch.int32, device="cuda")
        bb = torch.empty_like(bc)
        mto = torch.empty(e + 1, dtype=torch.int32, device="cuda")
        hk.tk_kernel.dispatch_expert_offsets(bc, t, counts, offs, bb, mto, None)
        perm = torch.empty(t * k, dtype=torch.int32, device="cuda")
        inv = torch.empty(t * k, dtype=torch.int32, device="cuda")
        hk.tk_kernel.dispatch_scatter(idx, offs, bb, perm, inv, None, None, None, None)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(idx), idx_ref)
        assert rel_err(_np(w), w_ref) <= 1e-6
        c_ref, o_ref = spec.expert_counts_offsets(idx_ref, e)
        np.testing.assert_array_equal(_np(counts), c_ref)
        np.testing.assert_array_equal(_np(offs), o_ref)
        p_ref, i_ref = spec.permutation(idx_ref, e)
        np.testing.assert_array_equal(_np(perm), p_ref)
        np.testing.assert_array_equal(_np(inv), i_ref)


@pytest.mark.parametrize("name", ["dsv3", "mixtral", "decode"])
def test_routing_full_size(hk, name):
    """Routing + offsets + permutation at the full configurations' T, E, k: bit-exact."""
    cfg = synth.CONFIGS[name]
    rng = np.random.default_rng(0)
    rng.standard_normal((1, 1))  # independent stream; shapes are what matters here
    logits = synth.make_logits(rng, cfg["T"], cfg["E"], cfg["skew"])
    t, e, k = cfg["T"], cfg["E"], cfg["k"]
    idx_ref, w_ref = spec.route_topk(logits, k)
    nblk = hk.tk_kernel.route_blocks(t)
    idx = torch.empty((t, k), dtype=torch.int32, device="cuda")
    w = torch.empty((t, k), dtype=torch.float32, device="cuda")
    bc = torch.empty((nblk, e), dtype=torch.int32, device="cuda")
    hk.tk_kernel.dispatch_route_topk(to_f32(logits), idx, w, bc)
    counts = torch.empty(e, dtype=torch.int32, device="cuda")
    offs = torch.empty(e + 1, dtype=torch.int32, device="cuda")
    bb = torch.empty_like(bc)
    mto = torch.empty(e + 1, dtype=torch.int32, device="cuda")
    hk.tk_kernel.dispatch_expert_offsets(bc, t, counts, offs, bb, mto, None)
    perm = torch.empty(t * k, dtype=torch.int32, device="cuda")
    inv = torch.empty(t * k, dtype=torch.int32, device="cuda")
    hk.tk_kernel.dispatch_scatter(idx, offs, bb, perm, inv, None, None, None, None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_np(idx), idx_ref)
    assert rel_err(_np(w), w_ref) <= 1e-6
    p_ref, i_ref = spec.permutation(idx_ref, e)
    np.testing.assert_array_equal(_np(perm), p_ref)
    np.testing.assert_array_equal(_np(inv), i_ref)
    assert _np(offs)[-1] == t * k


@pytest.mark.parametrize("t,e,k", [(70000, 8, 2), (512, 256, 8), (513, 256, 8), (1, 64, 8)])
def test_routing_block_bases(hk, t, e, k):
    """Block bases at both ends of the block-count range.  More than 2048
    routing blocks (T > 65536): each block-scan thread covers more block counts
    than it keeps in registers and reads them twice.  At most 16 blocks (T <=
    512): expert_offsets does the block scan itself; 17 blocks: the separate
    block scan.  Block counts, block bases, counts, offsets and the
    permutation: bit-exact against the oracle (block_base = exclusive prefix
    of an expert's counts over the 32-token routing blocks)."""
    rng = np.random.default_rng(11)
    logits = rng.standard_normal((t, e)).astype(np.float32)
    idx_ref, w_ref = spec.route_topk(logits, k)
    nblk = hk.tk_kernel.route_blocks(t)
    assert nblk == (t + 31) // 32
    print(f"routing T={t} E={e} k={k}: {nblk} blocks", flush=True)
    idx = torch.empty((t, k), dtype=torch.int32, device="cuda")
    w = torch.empty((t, k), dtype=torch.float32, device="cuda")
    bc = torch.empty((nblk, e), dtype=torch.int32, device="cuda")
    hk.tk_kernel.dispatch_route_topk(to_f32(logits), idx, w, bc)
    counts = torch.empty(e, dtype=torch.int32, device="cuda")
    offs = torch.empty(e + 1, dtype=torch.int32, device="cuda")
    bb = torch.full_like(bc, -1)
    mto = torch.empty(e + 1, dtype=torch.int32, device="cuda")
    hk.tk_kernel.dispatch_expert_offsets(bc, t, counts, offs, bb, mto, None)
    perm = torch.empty(t * k, dtype=torch.int32, device="cuda")
    inv = torch.empty(t * k, dtype=torch.int32, device="cuda")
    hk.tk_kernel.dispatch_scatter(idx, offs, bb, perm, inv, None, None, None, None)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_np(idx), idx_ref)
    assert rel_err(_np(w), w_ref) <= 1e-6
    blk = np.repeat(np.arange(nblk), 32)[:t]
    bc_ref = np.zeros((nblk, e), np.int64)
    for j in range(k):
        np.add.at(bc_ref, (blk, idx_ref[:, j]), 1)
    np.testing.assert_array_equal(_np(bc), bc_ref)
    bb_ref = np.cumsum(bc_ref, axis=0) - bc_ref
    np.testing.assert_array_equal(_np(bb), bb_ref)
    c_ref, o_ref = spec.expert_counts_offsets(idx_ref, e)
    np.testing.assert_array_equal(_np(counts), c_ref)
    np.testing.assert_array_equal(_np(offs), o_ref)
    p_ref, i_ref = spec.permutation(idx_ref, e)
    np.testing.assert_array_equal(_np(perm), p_ref)
    np.testing.assert_array_equal(_np(inv), i_ref)


def test_quantisers_bit_exact(hk):
    rng = np.random.default_rng(9)
    x = (rng.standard_normal((256, 384)) * 3).astype(np.float32)
    x[5, :128] = 0.0  # an all-zero group -> scale 1.0
    q, s = hk.quant_group(to_f32(x))
    q_ref, s_ref = spec.quant_group_1x128(x)
    np.testing.assert_array_equal(f8_np(q), q_ref)
    np.testing.assert_array_equal(_np(s), s_ref)
    w = rng.standard_normal((3, 256, 384)).astype(np.float32)
    q, s = hk.quant_block(to_f32(w))
    q_ref, s_ref = spec.quant_block_128x128(w)
    np.testing.assert_array_equal(f8_np(q), q_ref)
    np.testing.assert_array_equal(_np(s), s_ref)
    q, s = hk.quant_tensor(to_f32(x))
    q_ref, s_ref = spec.quant_per_tensor(x)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(f8_np(q), q_ref)
    assert _np(s)[0] == s_ref


def _golden(name):
    import os
    return np.load(os.path.join(os.path.dirname(__file__), "golden", name), allow_pickle=False)


@pytest.mark.parametrize("name", ["moe_tensor_e4k2.npz", "moe_block_e8k3_skew.npz", "moe_block_t8_e12k8.npz"])
def test_golden_fixture_native(hk, name):
    """The native path on the committed fixtures: routing bit-exact, output <= 1e-2."""
    g = _golden(name)
    block = g["x_scale"].ndim == 2
    d = dict(x_q=g["x_q"], x_scale=g["x_scale"] if block else np.float32(g["x_scale"]), logits=g["logits"],
             w13_q=g["w13_q"], w13_s=g["w13_s"], w2_q=g["w2_q"], w2_s=g["w2_s"], k=int(g["k"]))
    gg = moe_inputs_to_gpu(d)
    r = _run_steps(hk, gg, keep_h=False)
    np.testing.assert_array_equal(_np(r["topk_idx"]), g["topk_idx"])
    np.testing.assert_array_equal(_np(r["offsets"]), g["offsets"])
    np.testing.assert_array_equal(_np(r["perm"]), g["perm"])
    np.testing.assert_array_equal(_np(r["inv_perm"]), g["inv_perm"])
    assert rel_err(_np(r["topk_w"]), g["topk_w"]) <= 1e-6
    assert rel_err(bf16_np(r["out"]), g["out"].astype(np.float32)) <= TOL


def test_golden_dense_native(hk):
    g = _golden("dense_m64_n256_k256.npz")
    c = hk.gemm_fp8(to_f8(g["a_q"]), to_f8(g["b_q"]), to_f32([g["sa"]]), to_f32([g["sb"]]), out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert rel_err(c.cpu().numpy(), g["c_f32"]) <= 1e-4  # fp32 out: scale applied after vs before the sum
