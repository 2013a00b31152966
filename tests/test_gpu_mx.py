"""MX (1x32 e8m0) FP8 through the native path vs the oracle (oracle/mx.py).

Bars: quantiser (e4m3 bytes and e8m0 exponents) and scale packing bit-exact;
the GEMM bit-exact on +-1 known-answer inputs whose fp32 sums are exact (this
pins which exponent byte scales which operand lane), and on random N(0, 0.5)
operands within the reference's own tolerance |C - C_ref| <= 0.001 * max|C_ref|
for fp32 output (kernels/cdna4/gemm/mxfp8/MXFP8_4wave/4_wave.cu:501-506),
max relative error <= 1e-2 for bf16 output.
"""
import numpy as np
import pytest
import torch

from helpers import bf16_np, f8_np, rel_err, to_f8, to_f32
from oracle import fp8, mx

pytestmark = pytest.mark.gpu


def _u8(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint8)).cuda()


def _words(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).cuda()


def _edge_input(rng, r, c):
    x = (rng.standard_normal((r, c)) * np.exp2(rng.integers(-30, 30, (r, 1)))).astype(np.float32)
    if r >= 8 and c >= 128:
        x[0] = 0.0                                                  # all-zero blocks
        x[1, :32] = np.float32(2.0) ** -130                         # subnormal amax -> e8m0 0
        x[2, :32] = np.float32(1.9999999)                           # just below a power of two
        x[2, 32:64] = np.float32(2.0)                               # exactly a power of two
        x[3, :32] = np.float32(3.0e38)                              # large magnitudes
        x[4, :32] = rng.standard_normal(32).astype(np.float32) * np.float32(1e-30)
        x[4, 0] = np.float32(1e6)                                   # small elements under a big amax
        x[5, 64:96] = np.float32(2.0) ** -126                       # smallest normal amax
        x[6, :] = -np.abs(x[6, :])                                  # negative block maxima
    return x


@pytest.mark.parametrize("r,c", [(1, 32), (7, 96), (64, 128), (300, 4096), (2048, 7168)])
def test_quant_mx_bit_exact(hk, r, c):
    rng = np.random.default_rng(r * 7 + c)
    x = _edge_input(rng, r, c)
    q_ref, s_ref = mx.quant_mx(x)
    q, s = hk.quant_mx(to_f32(x))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(f8_np(q), q_ref)


@pytest.mark.parametrize("rows,k", [(1, 128), (64, 128), (70, 256), (300, 4096), (8192, 7168)])
def test_mx_pack_scales_bit_exact(hk, rows, k):
    rng = np.random.default_rng(rows + k)
    s = rng.integers(0, 255, (rows, k // 32), dtype=np.uint8)
    p = hk.mx_pack_scales(_u8(s))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(p.cpu().numpy().view(np.uint32), mx.mx_pack_scales(s))


def _pm1_mx(rng, rows, k):
    q = np.where(rng.integers(0, 2, (rows, k)) == 1, 0x38, 0xB8).astype(np.uint8)
    s = rng.integers(124, 131, (rows, k // 32)).astype(np.uint8)
    return q, s


@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (512, 512, 1024), (77, 256, 384), (1, 256, 128),
                                   (300, 768, 2048)])
def test_gemm_mx_known_answer_fp32(hk, m, n, k):
    """+-1 elements, exponents 124..130: every product is +-2^j (|j| <= 6) and
    every fp32 sum is exact, so the output must match bit for bit."""
    rng = np.random.default_rng(m * 3 + n + k)
    a, sa = _pm1_mx(rng, m, k)
    b, sb = _pm1_mx(rng, n, k)
    ref = mx.gemm_mx(a, sa, b, sb)
    c = hk.gemm_mx(to_f8(a), _words(mx.mx_pack_scales(sa)), to_f8(b), _words(mx.mx_pack_scales(sb)),
                   out_dtype=torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(c.cpu().numpy(), ref)


@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (100, 512, 640), (1000, 256, 2048), (33, 1024, 128)])
def test_gemm_mx_random(hk, m, n, k):
    d = mx.make_mx_dense(m, n, k, seed=m + k)
    ref = mx.gemm_mx(d["a_q"], d["sa"], d["b_q"], d["sb"])
    args = (to_f8(d["a_q"]), _words(mx.mx_pack_scales(d["sa"])), to_f8(d["b_q"]),
            _words(mx.mx_pack_scales(d["sb"])))
    c32 = hk.gemm_mx(*args, out_dtype=torch.float32)
    c16 = hk.gemm_mx(*args, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    got = c32.cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-3 * np.abs(ref).max()
    assert rel_err(bf16_np(c16), ref) <= 1e-2
    # bf16 output is the RNE rounding of the fp32 result
    np.testing.assert_array_equal(bf16_np(c16), fp8.bf16_round(got))


def test_mx_pipeline_quant_pack_gemm(hk):
    """fp32 operands -> device quantiser -> device packing -> MX GEMM, against
    the oracle run on the same fp32 inputs."""
    rng = np.random.default_rng(9)
    a = (rng.standard_normal((384, 1024)) * 0.5).astype(np.float32)
    b = (rng.standard_normal((512, 1024)) * 0.5).astype(np.float32)
    a[5] *= 1e4  # rows of very different magnitude
    b[7] *= 1e-4
    a_q, sa = hk.quant_mx(to_f32(a))
    b_q, sb = hk.quant_mx(to_f32(b))
    c = hk.gemm_mx(a_q, hk.mx_pack_scales(sa), b_q, hk.mx_pack_scales(sb), out_dtype=torch.float32)
    torch.cuda.synchronize()
    ra, rsa = mx.quant_mx(a)
    rb, rsb = mx.quant_mx(b)
    ref = mx.gemm_mx(ra, rsa, rb, rsb)
    got = c.cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-3 * np.abs(ref).max()
    # per row, relative to that row's own scale (rows differ by 1e8 in magnitude)
    row_max = np.abs(ref).max(1, keepdims=True)
    assert np.all(np.abs(got - ref) <= 1e-3 * row_max + 1e-30)


def test_gemm_mx_reference_shape_8192(hk):
    """The reference harness's shape, M = N = K = 8192 (4_wave.cu:23), N(0, 0.5)
    operands quantised on the device; rows checked on a seeded sample against
    the oracle, plus the column-sum identity over the whole output."""
    g = torch.Generator(device="cuda").manual_seed(42)
    a = torch.randn((8192, 8192), generator=g, device="cuda") * 0.5
    b = torch.randn((8192, 8192), generator=g, device="cuda") * 0.5
    a_q, sa = hk.quant_mx(a)
    b_q, sb = hk.quant_mx(b)
    del a, b
    c = hk.gemm_mx(a_q, hk.mx_pack_scales(sa), b_q, hk.mx_pack_scales(sb), out_dtype=torch.float32)
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(1).choice(8192, 64, replace=False))
    aq, san = f8_np(a_q), sa.cpu().numpy()
    bq, sbn = f8_np(b_q), sb.cpu().numpy()
    ref = mx.gemm_mx(aq[rows], san[rows], bq, sbn)
    got = c[torch.from_numpy(rows).cuda()].cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-3 * np.abs(ref).max()
    # column sums: sum_m C[m, :] = (sum_m deq(A)[m, :]) . deq(B)^T
    colsum = c.double().sum(0).cpu().numpy()
    asum = mx.dequant_mx(aq, san).sum(0)
    want = mx.dequant_mx(bq, sbn) @ asum
    # fp32 rounding of 8192 rows, summed: far below a misapplied exponent
    assert np.abs(colsum - want).max() <= 1e-4 * np.sqrt(8192) * np.abs(ref).max()
