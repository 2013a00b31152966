"""The per-token layer reference used by the full-shape GPU tests
(helpers.sampled_layer_reference) equals the oracle's permuted, grouped
pipeline (spec.moe_forward) on every token of small cases."""
import numpy as np
import pytest

from helpers import sampled_layer_reference
from oracle import spec, synth


@pytest.mark.parametrize("block,skew", [(True, True), (False, False), (True, False)])
def test_sampled_reference_matches_the_oracle(block, skew):
    d = synth.make_moe(T=37, H=256, I=256, E=6, k=3, block=block, skew=skew, seed=5)
    ref = spec.moe_forward(d["x_q"], d["x_scale"], d["logits"], d["w13_q"], d["w13_s"], d["w2_q"], d["w2_s"],
                           d["k"], return_all=True)
    toks = np.arange(37)
    xs = d["x_scale"][toks] if block else d["x_scale"]
    got = sampled_layer_reference(toks, ref["topk_idx"], ref["topk_w"], d["x_q"][toks], xs,
                                  lambda e: d["w13_q"][e], lambda e: d["w13_s"][e],
                                  lambda e: d["w2_q"][e], lambda e: d["w2_s"][e], block,
                                  h_scale=None if block else ref["hs"])
    # same arithmetic; only the BLAS blocking of the per-expert products may differ
    assert spec.rel_err(got, ref["out_f32"]) <= 1e-5
