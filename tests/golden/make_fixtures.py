"""Write the golden fixtures under tests/golden/ (run from the repository root:
``python tests/golden/make_fixtures.py``).

The reference has no MoE implementation and no golden vectors for this path,
so these fixtures freeze the oracle's outputs (oracle/spec.py) on small seeded
inputs: any later change to the specification or to its numerics shows up as
a fixture mismatch in tests/test_oracle.py.  Inputs come from oracle/synth.py.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import mx, spec, synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

MOE_CASES = {
    "moe_tensor_e4k2": dict(T=48, H=256, I=128, E=4, k=2, block=False, skew=False, seed=21),
    "moe_block_e8k3_skew": dict(T=40, H=256, I=128, E=8, k=3, block=True, skew=True, seed=22),
    "moe_block_t8_e12k8": dict(T=8, H=256, I=128, E=12, k=8, block=True, skew=False, seed=23),
}


def main():
    d = synth.make_dense(64, 256, 256, seed=20)
    c = spec.gemm_fp8(d["a_q"], d["b_q"], d["sa"], d["sb"], out="f32")
    np.savez_compressed(os.path.join(OUT, "dense_m64_n256_k256.npz"), a_q=d["a_q"], b_q=d["b_q"],
                        sa=np.float32(d["sa"]), sb=np.float32(d["sb"]), c_f32=c)
    # MX: fp32 operands -> e8m0 exponents, e4m3 bytes, packed words, fp32 C
    d = mx.make_mx_dense(96, 256, 256, seed=24)
    np.savez_compressed(os.path.join(OUT, "mx_m96_n256_k256.npz"), mx_a=d["a"], mx_b=d["b"], a_q=d["a_q"],
                        sa=d["sa"], b_q=d["b_q"], sb=d["sb"], sa_packed=mx.mx_pack_scales(d["sa"]),
                        sb_packed=mx.mx_pack_scales(d["sb"]),
                        c_f32=mx.gemm_mx(d["a_q"], d["sa"], d["b_q"], d["sb"]))
    for name, cfg in MOE_CASES.items():
        cfg = dict(cfg)
        seed = cfg.pop("seed")
        m = synth.make_moe(seed=seed, **cfg)
        r = spec.moe_forward(m["x_q"], m["x_scale"], m["logits"], m["w13_q"], m["w13_s"], m["w2_q"],
                             m["w2_s"], m["k"], return_all=True)
        np.savez_compressed(
            os.path.join(OUT, name + ".npz"), x_q=m["x_q"], x_scale=np.asarray(m["x_scale"], np.float32),
            logits=m["logits"], w13_q=m["w13_q"], w13_s=m["w13_s"], w2_q=m["w2_q"], w2_s=m["w2_s"],
            k=np.int32(m["k"]), topk_idx=r["topk_idx"], topk_w=r["topk_w"], counts=r["counts"],
            offsets=r["offsets"], perm=r["perm"], inv_perm=r["inv_perm"], hq=r["hq"], out=r["out"])
    print("fixtures written to", OUT)


if __name__ == "__main__":
    main()
