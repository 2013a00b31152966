"""The MoE layers replayed from a captured HIP graph vs the same calls run eagerly.

Every kernel of hkmoe_moe_forward / hkmoe_moe_forward_mx goes to torch's current
stream; the calls allocate nothing (caller-owned output and workspace), make no
host synchronisation, and clear their tile counters inside a kernel (no
hipMemsetAsync).  So one layer call can be captured once and replayed with new
inputs copied into the captured input tensors.

Bar: every replay equals the eager call on the same inputs, bit for bit.  Each
input set is replayed twice; between replays the test runs other eager work
(copies, and an eager call of the same layer object, on the same workspace, on
other inputs) and synchronises, and that eager result is checked as well.

The narrow path (block scales, even H/128 and I/128) forks to the library's
auxiliary stream and joins back through events; under capture the auxiliary
stream joins the graph the same way, with the late join (wide_share 2) and
without it (1).  Where T*k <= 2*E*max_rows it stays on the caller's stream,
which the capture takes as it is.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

T, H, I, E, K = 300, 768, 384, 64, 8
N_SETS = 3


def _logits(gen):
    lg = torch.randn((T, E), generator=gen, device="cuda")
    rank = torch.randperm(E, generator=gen, device="cuda").float() + 1.0
    return lg - 1.1 * torch.log(rank)[None, :]  # skewed: some experts get no tokens


def _capture(fn):
    """Warm up on a side stream (workspace, kernel attributes), then capture."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()
    return graph


def _same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def _replay_and_check(layer, sets):
    """sets: list of input tuples for layer(*inputs); returns nothing, asserts."""
    eager = [layer(*s).clone() for s in sets]
    torch.cuda.synchronize()
    static_in = [t.clone() for t in sets[0]]
    out = torch.empty_like(eager[0])
    graph = _capture(lambda: layer(*static_in, out=out))
    for rep in range(2):
        for i, s in enumerate(sets):
            for dst, src in zip(static_in, s):
                dst.copy_(src)
            graph.replay()
            torch.cuda.synchronize()
            assert _same(out, eager[i]), f"replay {rep} of input set {i} differs from the eager call"
            j = (i + 1) % len(sets)
            other = layer(*sets[j])
            torch.cuda.synchronize()
            assert _same(other, eager[j]), f"eager call on set {j} after a replay differs"
    # the output of a replay does not depend on what the previous replay left
    assert (out.float().abs().sum() > 0).item()


@pytest.mark.parametrize("block", [True, False])
def test_moe_layer_graph_replay(hk, block):
    gen = torch.Generator(device="cuda").manual_seed(123 + block)
    if block:
        w13_q, w13_s = hk.quant_block(torch.randn((E, 2 * I, H), generator=gen, device="cuda"))
        w2_q, w2_s = hk.quant_block(torch.randn((E, H, I), generator=gen, device="cuda"))
    else:
        q13, s13, q2, s2 = [], [], [], []
        for _ in range(E):
            q, s = hk.quant_tensor(torch.randn((2 * I, H), generator=gen, device="cuda"))
            q13.append(q); s13.append(s)
            q, s = hk.quant_tensor(torch.randn((H, I), generator=gen, device="cuda"))
            q2.append(q); s2.append(s)
        w13_q, w13_s = torch.stack(q13), torch.cat(s13)
        w2_q, w2_s = torch.stack(q2), torch.cat(s2)
    layer = hk.MoELayer(w13_q, w13_s, w2_q, w2_s, K)
    sets = []
    for _ in range(N_SETS):
        x = torch.randn((T, H), generator=gen, device="cuda")
        x_q, x_s = hk.quant_group(x) if block else hk.quant_tensor(x)
        sets.append((x_q, x_s, _logits(gen)))
    _replay_and_check(layer, sets)


def test_moe_layer_mx_graph_replay(hk):
    gen = torch.Generator(device="cuda").manual_seed(321)
    w13_q, w13_e = hk.quant_mx(torch.randn((E * 2 * I, H), generator=gen, device="cuda"))
    w2_q, w2_e = hk.quant_mx(torch.randn((E * H, I), generator=gen, device="cuda"))
    layer = hk.MoELayerMX(w13_q.view(E, 2 * I, H), w13_e.view(E, 2 * I, H // 32),
                          w2_q.view(E, H, I), w2_e.view(E, H, I // 32), K)
    sets = []
    for _ in range(N_SETS):
        x_q, x_e = hk.quant_mx(torch.randn((T, H), generator=gen, device="cuda"))
        sets.append((x_q, x_e, _logits(gen)))
    _replay_and_check(layer, sets)


@pytest.mark.parametrize("share,max_rows", [(1, 16), (2, 16), (1, 32)])
def test_moe_layer_graph_replay_narrow(hk, share, max_rows):
    """Block-scaled layer with experts of both kinds (<= max_rows rows: narrow
    kernel; larger: 256x256) captured with the narrow path on.  T*k = 1200:
    above 2*E*16 = 1024 the narrow kernels run on the auxiliary stream (with
    share 2 also the late join), at or below 2*E*32 = 2048 on the caller's
    stream after the 256x256 ones."""
    t, h, i, e, k = 300, 512, 256, 32, 4
    saved = hk.tk_kernel.get_narrow()
    hk.tk_kernel.set_narrow(16, max_rows, share)
    try:
        gen = torch.Generator(device="cuda").manual_seed(77 + share)
        w13_q, w13_s = hk.quant_block(torch.randn((e, 2 * i, h), generator=gen, device="cuda"))
        w2_q, w2_s = hk.quant_block(torch.randn((e, h, i), generator=gen, device="cuda"))
        layer = hk.MoELayer(w13_q, w13_s, w2_q, w2_s, k)
        sets = []
        for _ in range(N_SETS):
            x_q, x_s = hk.quant_group(torch.randn((t, h), generator=gen, device="cuda"))
            lg = torch.randn((t, e), generator=gen, device="cuda")
            rank = torch.randperm(e, generator=gen, device="cuda").float() + 1.0
            lg = lg - 1.1 * torch.log(rank)[None, :]
            sets.append((x_q, x_s, lg))
            r = hk.moe_forward_steps(x_q, x_s, lg, layer.w13_q, w13_s, layer.w2_q, w2_s, k, packed=True,
                                     narrow=(16, max_rows, share))
            torch.cuda.synchronize()
            counts = r["counts"].cpu()
            assert int(r["narrow_info"][0]) > 0 and (counts > max_rows).any()
        _replay_and_check(layer, sets)
    finally:
        hk.tk_kernel.set_narrow(*saved)
