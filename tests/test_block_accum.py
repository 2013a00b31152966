"""How the grouped GEMMs fold 128x128 / 1x128 block scales into the fp32
accumulator, emulated on the CPU with numpy.

Each v_mfma_f32_16x16x128 covers exactly one 128-wide K block, so the kernels
(gemm_fp8.hpp ``fold_block``, used by both the 256x256 and the narrow kernel)
start every MFMA from zero and fold its raw product P_k in with one fused
multiply-add per element:

    C <- fma(P_k, s_a[row, k] * s_w[col block, k], C)

The emulation below restates that in fp32 and checks it against the oracle
(``spec.gemm1_silu``'s dequantise-then-fp32 matmul) on rows whose 1x128 groups
have scales far apart: a normal group, an all-zero group (scale 1.0) and a
group near the fp32 floor (scale 2^-126), the pattern that overflowed the
earlier "rescale before the MFMA" recurrence
    u_k = u_{k-1} * (s_{k-1} / s_k) + P_k,   C = u_last * s_last,
which is emulated too, as a planted mistake, to show the case catches it.
"""
import numpy as np

from oracle import fp8, spec

GROUP = 128


def _raw_products(a_q, w_q):
    """P[k] [M, N]: the fp32 product of one K block of the e4m3 codes, as one
    MFMA returns it (exact sums of e4m3 products, rounded once to fp32)."""
    a = fp8.e4m3_to_f32(a_q).astype(np.float64)
    w = fp8.e4m3_to_f32(w_q).astype(np.float64)
    kb = a.shape[1] // GROUP
    return [(a[:, k * GROUP:(k + 1) * GROUP] @ w[:, k * GROUP:(k + 1) * GROUP].T).astype(np.float32)
            for k in range(kb)]


def fold_fma(a_q, a_s, w_q, w_s):
    """The kernels' block-scale accumulation (one fp32 FMA per element and K
    block, factor fl(s_a * s_w))."""
    P = _raw_products(a_q, w_q)
    m, n = P[0].shape
    c = np.zeros((m, n), np.float32)
    for k, pk in enumerate(P):
        f = (a_s[:, k:k + 1] * w_s[None, :, k]).astype(np.float32)  # [M, N] via the column block
        # fp32 FMA: the product is exact in float64 for fp32 inputs, one rounding
        c = (pk.astype(np.float64) * f.astype(np.float64) + c.astype(np.float64)).astype(np.float32)
    return c


def fold_rescale(a_q, a_s, w_q, w_s):
    """The earlier recurrence u_k = u_{k-1} * (s_{k-1}/s_k) + P_k (planted mistake)."""
    P = _raw_products(a_q, w_q)
    m, n = P[0].shape
    u = np.zeros((m, n), np.float32)
    prev = np.zeros((m, n), np.float32)
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        for k, pk in enumerate(P):
            s = (a_s[:, k:k + 1] * w_s[None, :, k]).astype(np.float32)
            u = (u * (prev / s) + pk).astype(np.float32)
            prev = s
        return (u * prev).astype(np.float32)


def _extreme_rows(rng, m, groups):
    """Activation rows with groups [N(0,1) | 0 | N(0,1)*1e-36 | N(0,1) ...]."""
    x = rng.standard_normal((m, groups * GROUP)).astype(np.float32)
    x[:, GROUP:2 * GROUP] = 0.0
    x[:, 2 * GROUP:3 * GROUP] *= np.float32(1e-36)
    return x


def _weights(rng, n, k):
    w = rng.standard_normal((1, n, k)).astype(np.float32)
    w_q, w_s = spec.quant_block_128x128(w)
    # per-128-row block of columns: [N, K/128] scales for the emulation
    w_s_cols = np.repeat(w_s[0], GROUP, axis=0)
    return w_q[0], w_s[0], w_s_cols


def test_scales_span_the_fp32_range():
    rng = np.random.default_rng(0)
    x = _extreme_rows(rng, 4, 4)
    _, s = spec.quant_group_1x128(x)
    assert np.all(s[:, 1] == 1.0)                  # all-zero group
    assert np.all(s[:, 2] == np.float32(2.0 ** -126))  # floored tiny group
    assert np.all((s[:, 0] > 1e-3) & (s[:, 0] < 1e-1))


def test_fold_fma_matches_the_oracle_on_extreme_scales():
    rng = np.random.default_rng(1)
    m, n, groups = 32, 256, 4
    x = _extreme_rows(rng, m, groups)
    a_q, a_s = spec.quant_group_1x128(x)
    w_q, w_s, w_s_cols = _weights(rng, n, groups * GROUP)
    ref = spec.grouped_gemm(a_q, a_s, w_q[None], w_s[None], np.array([0, m], np.int32))
    got = fold_fma(a_q, a_s, w_q, w_s_cols)
    assert np.all(np.isfinite(got))
    assert spec.rel_err(got, ref) <= 1e-5


def test_earlier_recurrence_overflows_on_the_same_rows():
    """The planted mistake (the earlier kernel arithmetic) gives inf / NaN where
    the oracle's result is finite and of ordinary size: the extreme-scale
    cases of the GPU tests exercise exactly this."""
    rng = np.random.default_rng(1)
    m, n, groups = 32, 256, 4
    x = _extreme_rows(rng, m, groups)
    a_q, a_s = spec.quant_group_1x128(x)
    w_q, w_s, w_s_cols = _weights(rng, n, groups * GROUP)
    ref = spec.grouped_gemm(a_q, a_s, w_q[None], w_s[None], np.array([0, m], np.int32))
    assert np.all(np.isfinite(ref)) and np.abs(ref).max() < 1e4
    bad = fold_rescale(a_q, a_s, w_q, w_s_cols)
    assert not np.all(np.isfinite(bad))


def test_fold_fma_matches_the_oracle_on_ordinary_rows():
    rng = np.random.default_rng(2)
    m, n, k = 48, 256, 7 * GROUP
    x = rng.standard_normal((m, k)).astype(np.float32)
    a_q, a_s = spec.quant_group_1x128(x)
    w_q, w_s, w_s_cols = _weights(rng, n, k)
    ref = spec.grouped_gemm(a_q, a_s, w_q[None], w_s[None], np.array([0, m], np.int32))
    assert spec.rel_err(fold_fma(a_q, a_s, w_q, w_s_cols), ref) <= 1e-5
    assert spec.rel_err(fold_rescale(a_q, a_s, w_q, w_s_cols), ref) <= 1e-5
