"""Dense FP8 GEMM (configs 1 and 4) through the native path vs the oracle.

Tolerance: max|C_gpu - C_ref| / max|C_ref| <= 1e-2 with C_ref the fp32
dequantised product (bf16 output) -- and exact equality for the +-1
known-answer test, whose fp32 result is an integer sum (the reference's KAT,
kernels/cdna3/gemm/fp8fp32/mi300x/8192_256_256_64_32/data_logs/
0613_003858_outputs/test_python.py:8-12).
"""
import numpy as np
import pytest
import torch

from helpers import bf16_np, rel_err, to_f8, to_f32
from oracle import fp8, spec, synth

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _pm1(rng, shape):
    return np.where(rng.integers(0, 2, shape) == 1, 0x38, 0xB8).astype(np.uint8)  # +1 / -1


@pytest.fixture
def dense_mfma(hk, request):
    """MFMA shape of the 128x128-tile dense kernel for one test (16x16x128 or
    32x32x64), restored afterwards."""
    saved = hk.tk_kernel.get_dense_mfma()
    hk.tk_kernel.set_dense_mfma(request.param)
    yield request.param
    hk.tk_kernel.set_dense_mfma(saved)


# all four shapes have fewer 256x256 tiles than two per CU: the 128x128 kernel
@pytest.mark.parametrize("dense_mfma", [16, 32], indirect=True)
@pytest.mark.parametrize("m,n,k", [(256, 256, 128), (512, 512, 1024), (2048, 2048, 2048), (77, 256, 384)])
def test_pm1_known_answer_fp32(hk, dense_mfma, m, n, k):
    """+-1 operands: every output is an exact integer; fp32 output must match bit
    for bit, with either MFMA shape of the small-problem kernel."""
    rng = np.random.default_rng(m + n + k)
    a = _pm1(rng, (m, k))
    b = _pm1(rng, (n, k))
    ref = fp8.e4m3_to_f32(a) @ fp8.e4m3_to_f32(b).T
    c = torch.empty((m, n), dtype=torch.float32, device="cuda")
    hk.tk_kernel.dispatch_micro(to_f8(a), to_f8(b), c)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(c.cpu().numpy(), ref)


@pytest.mark.parametrize("dense_mfma", [32], indirect=True)
@pytest.mark.parametrize("m,n,k", [(1, 256, 128), (300, 768, 640), (2048, 2048, 2048)])
def test_gemm_mfma32_bf16(hk, dense_mfma, m, n, k):
    """The 32x32x64 kernel with scales and bf16 output against the oracle, and
    against the 16x16x128 kernel's bf16 output (same fp32 sums up to order)."""
    d = synth.make_dense(m, n, k, seed=m + 1)
    ref = spec.gemm_fp8(d["a_q"], d["b_q"], d["sa"], d["sb"], out="f32")
    args = (to_f8(d["a_q"]), to_f8(d["b_q"]), to_f32([d["sa"]]), to_f32([d["sb"]]))
    c32 = hk.gemm_fp8(*args)
    hk.tk_kernel.set_dense_mfma(16)
    c16 = hk.gemm_fp8(*args)
    torch.cuda.synchronize()
    assert rel_err(bf16_np(c32), ref) <= TOL
    assert rel_err(bf16_np(c32), bf16_np(c16)) <= 8e-3


def test_dispatch_micro_4d_views(hk):
    """Reference call shape: A [1,1,M,K], B [1,1,N,K], C [1,1,M,N] fp32 (test_python.py:10-12)."""
    rng = np.random.default_rng(5)
    a = _pm1(rng, (256, 256))
    b = _pm1(rng, (512, 256))
    c = torch.zeros((1, 1, 256, 512), dtype=torch.float32, device="cuda")
    hk.tk_kernel.dispatch_micro(to_f8(a).view(1, 1, 256, 256), to_f8(b).view(1, 1, 512, 256), c)
    torch.cuda.synchronize()
    ref = fp8.e4m3_to_f32(a) @ fp8.e4m3_to_f32(b).T
    np.testing.assert_array_equal(c[0, 0].cpu().numpy(), ref)


@pytest.mark.parametrize("m,n,k", [(1, 256, 128), (100, 512, 256), (300, 768, 640), (1000, 256, 2048)])
def test_gemm_scaled_bf16_ragged(hk, m, n, k):
    d = synth.make_dense(m, n, k, seed=m)
    ref = spec.gemm_fp8(d["a_q"], d["b_q"], d["sa"], d["sb"], out="f32")
    c = hk.gemm_fp8(to_f8(d["a_q"]), to_f8(d["b_q"]), to_f32([d["sa"]]), to_f32([d["sb"]]))
    torch.cuda.synchronize()
    got = bf16_np(c)
    assert rel_err(got, ref) <= TOL
    # bf16 output is the RNE rounding of the fp32 result up to accumulation order
    assert rel_err(got, fp8.bf16_round(ref)) <= 8e-3


def test_config1_dense_2048(hk):
    d = synth.make("dense_2048", seed=0)
    ref = spec.gemm_fp8(d["a_q"], d["b_q"], d["sa"], d["sb"], out="f32")
    c = hk.gemm_fp8(to_f8(d["a_q"]), to_f8(d["b_q"]), to_f32([d["sa"]]), to_f32([d["sb"]]))
    torch.cuda.synchronize()
    assert rel_err(bf16_np(c), ref) <= TOL


def test_config4_tp_local_rows_sampled(hk):
    """Config 4 at full size (8192 x 8192 x 2048); rows checked on a seeded sample."""
    d = synth.make("tp_local", seed=0)
    c = hk.gemm_fp8(to_f8(d["a_q"]), to_f8(d["b_q"]), to_f32([d["sa"]]), to_f32([d["sb"]]))
    torch.cuda.synchronize()
    rows = np.sort(np.random.default_rng(1).choice(8192, 96, replace=False))
    ref = spec.gemm_fp8(d["a_q"][rows], d["b_q"], d["sa"], d["sb"], out="f32")
    got = bf16_np(c[torch.from_numpy(rows).cuda()])
    assert rel_err(got, ref) <= TOL
    # checksum of checksums over the full output (size-independent property):
    # column sums of C equal (sum_m A[m,:]) . B^T up to fp32 rounding
    colsum_ref = (spec.dequant_per_tensor(d["a_q"], d["sa"]).sum(0, dtype=np.float64)
                  @ spec.dequant_per_tensor(d["b_q"], d["sb"]).T.astype(np.float64))
    colsum = c.float().sum(0, dtype=torch.float64).cpu().numpy()
    assert rel_err(colsum, colsum_ref) <= TOL


def test_gemm_rejects_bad_shapes(hk):
    a = torch.zeros((64, 100), dtype=torch.float8_e4m3fn, device="cuda")
    b = torch.zeros((256, 100), dtype=torch.float8_e4m3fn, device="cuda")
    c = torch.zeros((64, 256), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 128"):
        hk.tk_kernel.dispatch_gemm_fp8(a, b, c)
    with pytest.raises(RuntimeError, match="contiguous"):
        hk.tk_kernel.dispatch_gemm_fp8(a.t(), b, c)
