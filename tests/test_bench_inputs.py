"""bench.py's MoE inputs come from the path's frozen synthetic generator.

bench.host_draw restates oracle/synth.py's first draws (x, logits, Zipf bias
permutation) because the benchmark may not import the oracle; these tests pin
the two together, so the benched routing is the specification's draw.
"""
import json
import os
import subprocess
import sys

import numpy as np
import pytest

import bench
from oracle import spec, synth


@pytest.mark.parametrize("name", ["dsv3", "mixtral", "decode"])
def test_host_draw_is_the_spec_draw(name):
    cfg = dict(bench.CONFIGS[name])
    E = min(cfg["E"], 24)
    small = dict(cfg, T=40, H=256, E=E)
    x, logits = bench.host_draw(small, seed=3)
    d = synth.make_moe(T=40, H=256, I=128, E=E, k=min(cfg["k"], E), block=cfg["block"], skew=cfg["skew"],
                       seed=3)
    np.testing.assert_array_equal(logits, d["logits"])
    x_q = spec.quant_group_1x128(x)[0] if cfg["block"] else spec.quant_per_tensor(x)[0]
    np.testing.assert_array_equal(x_q, d["x_q"])


def test_dsv3_draw_routing_profile():
    """The full-size config-3 draw (seed 0): skewed, with empty experts and a
    long tail of experts small enough for the narrow kernel."""
    cfg = bench.CONFIGS["dsv3"]
    _, logits = bench.host_draw(cfg, seed=0)
    idx, _ = spec.route_topk(logits, cfg["k"])
    counts = np.bincount(idx.ravel(), minlength=cfg["E"])
    assert counts.sum() == cfg["T"] * cfg["k"]
    assert (counts == 0).sum() == 69
    assert counts.max() == 7970
    assert ((counts > 0) & (counts <= 64)).sum() == 136


@pytest.mark.parametrize("n", [2, 8])
def test_bench_refuses_more_than_one_gpu(n):
    """--gpus N > 1 exits with status 2 and a one-line JSON message, before
    touching torch or the GPU (the build measures one GPU only)."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", str(n)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]
