"""Narrow path of the one-call layer (experts of <= 64 rows in the
weight-streaming kernel, on an auxiliary stream beside the 256x256 kernels, or
after them on the caller's stream when T*k <= 2*E*max_rows) against the
256x256 kernels.

The narrow kernel uses the 256x256 kernel's operand order, block-scale arithmetic
and epilogue, so the layer output is bit-identical with the narrow path off,
on, on a tiny grid (many items per workgroup), with a lower row threshold, and
with the narrow path's CUs joining the first 256x256 GEMM's tiles afterwards
(wide_share 2) or not (1).
With top-1 routing the combine is the identity (weight 1.0), so ``out`` is
GEMM 2's output ``y`` itself and those cases pin it bit for bit.  Shapes cover
prefetch depths 8, 4 and 2, items of one and of several groups of K steps,
both weight layouts, and configuration 3's hidden / expert sizes.
"""
import numpy as np
import pytest
import torch

from helpers import moe_inputs_to_gpu, rel_err
from oracle import spec, synth

pytestmark = pytest.mark.gpu

# name: T, H, I, E, k   (H/128 and I/128 set the prefetch depth and groups)
CASES = {
    "p8_g2_g1": dict(T=512, H=2048, I=1024, E=48, k=4),    # GEMM 1: 16 steps, GEMM 2: 8
    "p8_top1": dict(T=1024, H=1024, I=1024, E=64, k=1),    # 8 and 8 steps, out == y
    "p4_p2": dict(T=300, H=512, I=256, E=32, k=2),         # 4 and 2 steps
    "dsv3_shape": dict(T=256, H=7168, I=2048, E=32, k=8),  # 56 and 16 steps
}


@pytest.fixture
def narrow_restore(hk):
    saved = hk.tk_kernel.get_narrow()
    yield
    hk.tk_kernel.set_narrow(*saved)


def _dev_inputs(hk, T, H, I, E, k, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    dev = "cuda"
    x = torch.randn(T, H, device=dev, generator=gen)
    bias = torch.from_numpy(synth.skew_bias(np.random.default_rng(seed), E)).to(dev)
    logits = (torch.randn(T, E, device=dev, generator=gen) + bias[None, :]).contiguous()
    x_q, x_s = hk.quant_group(x)
    w13_q, w13_s = hk.quant_block(torch.randn(E, 2 * I, H, device=dev, generator=gen))
    w2_q, w2_s = hk.quant_block(torch.randn(E, H, I, device=dev, generator=gen))
    return dict(x_q=x_q, x_scale=x_s, logits=logits, w13_q=w13_q, w13_scale=w13_s, w2_q=w2_q,
                w2_scale=w2_s, top_k=k)


def _one_call(hk, g, w13, w2, packed):
    out = hk.moe_forward(g["x_q"], g["x_scale"], g["logits"], w13, g["w13_scale"], w2, g["w2_scale"],
                         g["top_k"], packed=packed)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("packed", [True, False])
@pytest.mark.parametrize("name", list(CASES))
def test_narrow_bit_exact(hk, narrow_restore, name, packed):
    c = CASES[name]
    g = _dev_inputs(hk, seed=31, **c)
    w13, w2 = g["w13_q"], g["w2_q"]
    if packed:
        w13, w2 = hk.pack_weights(w13, gate_up=True), hk.pack_weights(w2)
    steps = hk.moe_forward_steps(g["x_q"], g["x_scale"], g["logits"], w13, g["w13_scale"], w2,
                                 g["w2_scale"], g["top_k"], packed=packed)
    torch.cuda.synchronize()
    counts = steps["counts"].cpu().numpy()
    assert ((counts > 0) & (counts <= 64)).any(), "no expert for the narrow kernel"
    assert (counts > 64).any(), "no expert for the 256x256 kernel"
    print(f"{name} packed={packed}: {int(((counts > 0) & (counts <= 64)).sum())} narrow experts of "
          f"{int((counts > 0).sum())}", flush=True)

    hk.tk_kernel.set_narrow(0, 64, 0)
    off = _one_call(hk, g, w13, w2, packed).clone()
    assert torch.equal(off.view(torch.int16), steps["out"].view(torch.int16))
    # threshold 64: every case here has T*k <= 2*E*64 (one stream); threshold 16:
    # where T*k > 2*16*E (p8_g2_g1, dsv3_shape) the narrow kernels run on the
    # auxiliary stream, and with wide_share 2 their CUs also join the first
    # 256x256 GEMM's tiles (late join)
    print(f"  experts of 1..16 rows: {int(((counts > 0) & (counts <= 16)).sum())}", flush=True)
    # (4096, 64, 1): more CUs than the device has; the library keeps a quarter
    # of them for the first 256x256 GEMM
    for cus, max_rows, share in ((48, 64, 0), (3, 64, 0), (48, 16, 0), (40, 64, 1), (64, 64, 2), (3, 64, 1),
                                 (64, 16, 2), (3, 16, 2), (4096, 64, 1)):
        hk.tk_kernel.set_narrow(cus, max_rows, share)
        on = _one_call(hk, g, w13, w2, packed)
        assert torch.equal(on.view(torch.int16), off.view(torch.int16)), (cus, max_rows, share)
    if g["top_k"] == 1:
        # the combine is the identity: out is y, row for row
        y = steps["y"][steps["inv_perm"].long()]
        assert torch.equal(y.view(torch.int16), off.view(torch.int16))


@pytest.mark.parametrize("packed", [True, False])
@pytest.mark.parametrize("name", ["p8_g2_g1", "p4_p2"])
def test_split_steps_bit_exact(hk, name, packed):
    """The stepwise split (hkmoe_expert_offsets_narrow + hkmoe_grouped_gemm{1,2}_part
    on two streams) gives the 256x256-only intermediates bit for bit, and
    narrow_info holds the count of experts of 1..max_rows rows."""
    c = CASES[name]
    g = _dev_inputs(hk, seed=33, **c)
    w13, w2 = g["w13_q"], g["w2_q"]
    if packed:
        w13, w2 = hk.pack_weights(w13, gate_up=True), hk.pack_weights(w2)
    args = (g["x_q"], g["x_scale"], g["logits"], w13, g["w13_scale"], w2, g["w2_scale"], g["top_k"])
    ref = hk.moe_forward_steps(*args, packed=packed)
    for narrow in ((48, 64, 1), (5, 32, 0)):
        r = hk.moe_forward_steps(*args, packed=packed, narrow=narrow)
        torch.cuda.synchronize()
        counts = r["counts"].cpu()
        want = int(((counts > 0) & (counts <= narrow[1])).sum())
        assert int(r["narrow_info"][0]) == want and want > 0
        for key in ("hq", "hs", "y", "out"):
            assert torch.equal(r[key].view(torch.uint8), ref[key].view(torch.uint8)), (narrow, key)


def test_narrow_oracle(hk, narrow_restore):
    """A small skewed layer with the narrow path on vs the numpy oracle (<= 1e-2)."""
    d = synth.make_moe(T=200, H=512, I=256, E=24, k=3, block=True, skew=True, seed=41)
    g = moe_inputs_to_gpu(d)
    ref = spec.moe_forward(d["x_q"], d["x_scale"], d["logits"], d["w13_q"], d["w13_s"], d["w2_q"],
                           d["w2_s"], d["k"], return_all=True)
    counts = ref["counts"]
    assert ((counts > 0) & (counts <= 64)).any()
    hk.tk_kernel.set_narrow(8, 64, 0)
    out = _one_call(hk, g, g["w13_q"], g["w2_q"], False)
    assert rel_err(out.float().cpu().numpy(), ref["out_f32"]) <= 1e-2


def test_narrow_settings_checked(hk, narrow_restore):
    with pytest.raises(RuntimeError):
        hk.tk_kernel.set_narrow(-1, 64, 0)
    with pytest.raises(RuntimeError):
        hk.tk_kernel.set_narrow(8, 65, 0)
    with pytest.raises(RuntimeError):
        hk.tk_kernel.set_narrow(8, 64, 3)
    hk.tk_kernel.set_narrow(5, 32, 1)
    assert tuple(hk.tk_kernel.get_narrow()) == (5, 32, 1)
