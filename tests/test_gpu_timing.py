"""Per-dispatch kernel timing of the layer entry points (hkmoe_kernel_timing):
a timed layer call gives the same bits as an untimed one, and its timeline is
consistent: every kernel the schedule launches has an interval, the kernels on
the caller's stream follow one another in launch order, and the narrow
kernels (block scales) sit on the auxiliary stream beside the 256x256 GEMM 1.
"""
import pytest
import torch

from helpers import moe_inputs_to_gpu
from oracle import synth

pytestmark = pytest.mark.gpu


def _layer(hk, block, T=300, seed=5):
    d = synth.make_moe(T=T, H=512, I=256, E=16, k=4, block=block, skew=True, seed=seed)
    g = moe_inputs_to_gpu(d)
    layer = hk.MoELayer(g["w13_q"], g["w13_scale"], g["w2_q"], g["w2_scale"], g["top_k"])
    return layer, g


@pytest.mark.parametrize("block,T", [(True, 300), (False, 300), (True, 1000), (True, 64)])
def test_timed_calls_match_untimed(hk, block, T):
    """T=300: 10 routing blocks (the block scan runs inside expert_offsets) and,
    with block scales, T*k <= 2*E*64: the one-stream narrow schedule.  T=1000:
    32 blocks (separate block scan) and the two-stream schedule.  T=64: every
    expert has at most 64 rows, so only the narrow GEMMs are launched."""
    tk = hk.tk_kernel
    roles = tk.TIMING_ROLES
    layer, g = _layer(hk, block, T=T)
    want = layer(g["x_q"], g["x_scale"], g["logits"])
    torch.cuda.synchronize()
    tk.kernel_timing(3)
    try:
        outs = [layer(g["x_q"], g["x_scale"], g["logits"]) for _ in range(3)]
        torch.cuda.synchronize()
        sets = [tk.kernel_timing_read(i) for i in range(3)]
    finally:
        tk.kernel_timing(0)
    for o in outs:
        assert torch.equal(o.view(torch.int16), want.view(torch.int16))
    k, e = 4, 16
    fused_scan = tk.route_blocks(T) <= 16
    all_narrow = block and T <= 64
    one_stream = block and T * k <= 2 * e * 64
    for tl in sets:
        got = {roles[i]: v for i, v in enumerate(tl) if v[0] >= 0}
        print(f"block={block} T={T} timeline (ms): {got}", flush=True)
        expect = ["route_topk", "expert_offsets", "scatter", "combine"]
        expect += [] if all_narrow else ["grouped_gemm1", "grouped_gemm2"]
        expect += ["narrow_gemm1", "narrow_gemm2"] if block else []
        for name in expect:
            assert name in got, name
        assert ("expert_block_scan" in got) == (not fused_scan)
        if all_narrow:
            assert "grouped_gemm1" not in got and "grouped_gemm2" not in got
        assert got["route_topk"][0] == 0.0
        for b, e_ in got.values():
            assert 0.0 <= b < e_ < 1000.0
        main = [n for n in ("route_topk", "expert_block_scan", "expert_offsets", "scatter", "grouped_gemm1",
                            "requant", "grouped_gemm2", "combine") if n in got]
        for a, b in zip(main, main[1:]):
            assert got[a][1] <= got[b][0] + 1e-3, (a, b)
        assert ("requant" in got) == (not block)
        if one_stream:
            # after each 256x256 GEMM (when there is one), on the caller's stream
            seq = [n for n in ("grouped_gemm1", "narrow_gemm1", "grouped_gemm2", "narrow_gemm2", "combine")
                   if n in got]
            for a, b in zip(seq, seq[1:]):
                assert got[a][1] <= got[b][0] + 1e-3, (a, b)
        elif block:
            # beside the 256x256 GEMM 1 on the auxiliary stream, joined before the combine
            assert got["narrow_gemm1"][0] < got["grouped_gemm1"][1]
            assert got["narrow_gemm2"][1] <= got["combine"][0] + 1e-3


def test_timing_off_and_bad_sets(hk):
    tk = hk.tk_kernel
    tk.kernel_timing(0)
    with pytest.raises(RuntimeError):
        tk.kernel_timing_read(0)
    with pytest.raises(RuntimeError):
        tk.kernel_timing(-1)
    layer, g = _layer(hk, True, T=64)
    tk.kernel_timing(2)
    try:
        layer(g["x_q"], g["x_scale"], g["logits"])
        torch.cuda.synchronize()
        first = tk.kernel_timing_read(0)
        assert first[0][0] == 0.0
        # set 1 was not used yet: nothing recorded
        assert all(v == (-1.0, -1.0) for v in tk.kernel_timing_read(1))
        with pytest.raises(RuntimeError):
            tk.kernel_timing_read(2)
    finally:
        tk.kernel_timing(0)
