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


@pytest.mark.parametrize("block", [True, False])
def test_timed_calls_match_untimed(hk, block):
    tk = hk.tk_kernel
    roles = tk.TIMING_ROLES
    layer, g = _layer(hk, block)
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
    for tl in sets:
        got = {roles[i]: v for i, v in enumerate(tl) if v[0] >= 0}
        print(f"block={block} timeline (ms): {got}", flush=True)
        for name in ("route_topk", "expert_block_scan", "expert_offsets", "scatter", "grouped_gemm1",
                     "grouped_gemm2", "combine"):
            assert name in got, name
        assert got["route_topk"][0] == 0.0
        for b, e in got.values():
            assert 0.0 <= b < e < 1000.0
        main = [n for n in ("route_topk", "expert_block_scan", "expert_offsets", "scatter", "grouped_gemm1",
                            "requant", "grouped_gemm2", "combine") if n in got]
        for a, b in zip(main, main[1:]):
            assert got[a][1] <= got[b][0] + 1e-3, (a, b)
        assert ("requant" in got) == (not block)
        if block:
            # T*k = 1200 <= 2*E*64: the one-stream narrow schedule, after each 256x256 GEMM
            assert got["grouped_gemm1"][1] <= got["narrow_gemm1"][0] + 1e-3
            assert got["narrow_gemm1"][1] <= got["grouped_gemm2"][0] + 1e-3
            assert got["grouped_gemm2"][1] <= got["narrow_gemm2"][0] + 1e-3
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
