"""Pins for the MX (1x32 e8m0) part of the CPU oracle (no GPU).

  mx.e8m0_from_amax    floor(log2) in float64 (numpy library routine) over random
                       magnitudes and the edge cases (powers of two and their
                       float32 predecessors, subnormal, zero, the largest float)
  mx.quant_mx          torch.float8_e4m3fn casts (library) of the power-of-two
                       scaled blocks; closed form: every block with a normal amax
                       has its largest element quantised into [1, 2]
  mx.mx_pack_scales    the reference's two-step pack_scales_kernel +
                       repack_scales_for_mfma_kernel restatement (4_wave.cu:323-364)
                       and the scale_pipeline known-answer rule of
                       tests/unit/cdna4/warp/register/tile/mma_scaled.cu:70-96
  mx.gemm_mx           torch.matmul on operands dequantised by torch ops
                       (repeat_interleave of the exponents); the per-tensor GEMM
                       (spec.gemm_fp8, pinned elsewhere) when every exponent is 127;
                       a known-answer test with +-1 elements whose sums are exact
A final test plants mistakes in the MX oracle and checks that the pins catch them.
"""
import numpy as np
import torch

from oracle import fp8, mx, spec


# ----------------------------------------------------------------------------
# pins, written as checks so the planted-mistake test can reuse them
# ----------------------------------------------------------------------------
def _amax_cases(rng):
    pw = np.float32(2.0) ** np.arange(-126, 128, dtype=np.float32)
    below = np.nextafter(pw, np.float32(0))  # largest float32 below each power of two
    rand = (rng.standard_normal(20000) * np.exp2(rng.uniform(-140, 126, 20000))).astype(np.float32)
    edge = np.array([0.0, 1e-45, 1e-40, 1.17549435e-38, 1.0, 3.4028235e38, 448.0, 0.5], np.float32)
    return np.abs(np.concatenate([pw, below, rand, edge])).astype(np.float32)


def check_e8m0(m):
    a = _amax_cases(np.random.default_rng(1))
    got = m.e8m0_from_amax(a)
    with np.errstate(divide="ignore"):
        fl = np.floor(np.log2(a.astype(np.float64)))
    want = np.where(a > 0, np.clip(np.where(np.isfinite(fl), fl, -1e9) + 127, 0, 254), 0).astype(np.uint8)
    np.testing.assert_array_equal(got, want)


def check_quant(m):
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((37, 256)) * np.exp2(rng.integers(-20, 20, (37, 1)))).astype(np.float32)
    x[3] = 0.0                                   # all-zero row
    x[4, :32] = np.float32(2.0) ** -130          # subnormal block -> s = 0
    x[5, 32:64] = np.float32(3.0e38)             # near the top of float32
    q, s = m.quant_mx(x)
    assert s.shape == (37, 8) and q.shape == x.shape
    # e4m3 of the power-of-two scaled block, by the library cast
    sh = (127 - s.astype(np.int64)).repeat(32, axis=1)
    scaled = torch.from_numpy(np.ldexp(x.astype(np.float64), sh).astype(np.float32))
    want = scaled.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(q, want)
    # closed form: the block maximum lands in [1, 2] (amax normal)
    amax = np.abs(x).reshape(37, 8, 32).max(2)
    qmax = np.abs(fp8.e4m3_to_f32(q)).reshape(37, 8, 32).max(2)
    normal = amax >= np.float32(2.0) ** -126
    assert np.all((qmax[normal] >= 1.0) & (qmax[normal] <= 2.0))
    assert np.all(s[3] == 0) and np.all(q[3] == 0)
    assert s[4, 0] == 0


def check_pack(m):
    rng = np.random.default_rng(3)
    for rows, kb in ((64, 4), (128, 16), (192, 56)):
        s = rng.integers(0, 255, (rows, kb), dtype=np.uint8)
        it = m.pack_scales_iter(s)
        two_step = m.repack_scales_for_mfma(it)
        one_step = m.mx_pack_scales(s)
        np.testing.assert_array_equal(one_step, two_step)
        # scale_pipeline KAT: lane lid of the 64-row window at row_offset gets
        # byte k_sub = lid/16 of the iteration words of rows row_offset + 16g + lid%16
        for ki in range(kb // 4):
            for row_offset in range(0, rows, 64):
                for lid in range(64):
                    r16, k_sub = lid % 16, lid // 16
                    exp = 0
                    for g in range(4):
                        w = int(it[ki, row_offset + g * 16 + r16])
                        exp |= ((w >> (8 * k_sub)) & 0xFF) << (8 * g)
                    assert int(one_step[ki, row_offset + lid]) == exp
    # rows not a multiple of 64: padded rows read as 0, real rows as above
    s = rng.integers(1, 255, (70, 8), dtype=np.uint8)
    p = m.mx_pack_scales(s)
    assert p.shape == (2, 128)
    full = m.mx_pack_scales(np.vstack([s, np.zeros((58, 8), np.uint8)]))
    np.testing.assert_array_equal(p, full)


def _deq_torch(q, s):
    v = torch.from_numpy(fp8.e4m3_to_f32(q)).double()
    e = torch.from_numpy(s.astype(np.int64) - 127).repeat_interleave(32, dim=1)
    return v * torch.pow(torch.tensor(2.0, dtype=torch.float64), e.double())


def check_gemm(m):
    rng = np.random.default_rng(4)
    d = m.make_mx_dense(40, 48, 256, seed=5)
    got = m.gemm_mx(d["a_q"], d["sa"], d["b_q"], d["sb"])
    want = (_deq_torch(d["a_q"], d["sa"]) @ _deq_torch(d["b_q"], d["sb"]).T).float().numpy()
    assert spec.rel_err(got, want) <= 1e-6
    # all exponents 127: the per-tensor GEMM with unit scales
    a_q = d["a_q"]
    b_q = d["b_q"]
    ones_a = np.full(d["sa"].shape, 127, np.uint8)
    ones_b = np.full(d["sb"].shape, 127, np.uint8)
    got1 = m.gemm_mx(a_q, ones_a, b_q, ones_b)
    want1 = spec.gemm_fp8(a_q, b_q, np.float32(1), np.float32(1), out="f32")
    assert spec.rel_err(got1, want1) <= 1e-6
    # +-1 known answer: exponents 124..130 per (row, block), sums exact; the
    # reference's loop order (4_wave.cu:466-478), literally, on a tiny case
    M, N, K = 3, 5, 128
    a = np.where(rng.integers(0, 2, (M, K)) == 1, 0x38, 0xB8).astype(np.uint8)
    b = np.where(rng.integers(0, 2, (N, K)) == 1, 0x38, 0xB8).astype(np.uint8)
    sa = rng.integers(124, 131, (M, K // 32)).astype(np.uint8)
    sb = rng.integers(124, 131, (N, K // 32)).astype(np.uint8)
    af, bf = fp8.e4m3_to_f32(a), fp8.e4m3_to_f32(b)
    kat = np.zeros((M, N), np.float32)
    for i in range(M):
        for j in range(N):
            acc = np.float32(0)
            for kb in range(K // 32):
                fa = np.float32(2.0 ** (int(sa[i, kb]) - 127))
                fb = np.float32(2.0 ** (int(sb[j, kb]) - 127))
                for k in range(32):
                    acc = np.float32(acc + af[i, kb * 32 + k] * fa * bf[j, kb * 32 + k] * fb)
            kat[i, j] = acc
    np.testing.assert_array_equal(m.gemm_mx(a, sa, b, sb), kat)


# ----------------------------------------------------------------------------
def test_e8m0_vs_float64_log2():
    check_e8m0(mx)


def test_quant_mx_vs_torch_cast_and_closed_form():
    check_quant(mx)


def test_pack_one_step_vs_reference_two_step_and_kat():
    check_pack(mx)


def test_gemm_mx_vs_torch_and_known_answer():
    check_gemm(mx)


def test_planted_mx_mistakes_are_caught(monkeypatch):
    import pytest
    # (1) floor(log2) off by one (ceil-like)
    monkeypatch.setattr(mx, "e8m0_from_amax",
                        lambda a: np.where(np.asarray(a) > 0, np.clip(np.frexp(np.asarray(a, np.float64))[1] + 127, 0, 254),
                                           0).astype(np.uint8))
    with pytest.raises(AssertionError):
        check_e8m0(mx)
    with pytest.raises(AssertionError):
        check_quant(mx)
    monkeypatch.undo()
    # (2) g and k_sub swapped in the packing
    good_pack = mx.mx_pack_scales

    def bad_pack(s):
        w = good_pack(s)
        kt, r64 = w.shape
        t = w.reshape(kt, r64 // 64, 4, 16)
        b = np.stack([(t >> np.uint32(8 * g)) & np.uint32(0xFF) for g in range(4)], axis=-1)  # kt,tile,ksub,r16,g
        b = b.transpose(0, 1, 4, 3, 2)  # swap the roles of k_sub and g
        out = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16) | (b[..., 3] << 24)
        return out.reshape(kt, r64).astype(np.uint32)

    monkeypatch.setattr(mx, "mx_pack_scales", bad_pack)
    with pytest.raises(AssertionError):
        check_pack(mx)
    monkeypatch.undo()
    # (3) exponent applied with the wrong sign in the dequantisation
    good_deq = mx.dequant_mx
    monkeypatch.setattr(mx, "dequant_mx", lambda q, s: good_deq(q, (254 - s.astype(np.int64)).astype(np.uint8)))
    with pytest.raises(AssertionError):
        check_gemm(mx)
    monkeypatch.undo()
    # (4) B's exponents indexed by the A row (transposed scale operand)
    monkeypatch.setattr(mx, "gemm_mx", lambda a_q, sa, b_q, sb, out="f32": (
        mx.dequant_mx(a_q, sa) @ mx.dequant_mx(b_q, np.resize(sa, sb.shape)).T).astype(np.float32))
    with pytest.raises(AssertionError):
        check_gemm(mx)


# ----------------------------------------------------------------------------
# MX MoE layer oracle
# ----------------------------------------------------------------------------
def _pad_rows(a, n):
    out = np.zeros((n, a.shape[1]), dtype=a.dtype)
    out[:a.shape[0]] = a
    return out


def test_gather_words_tile_by_tile_vs_pack():
    """Each M tile's 256 words equal mx_pack_scales of that tile's rows (padded
    to 256 with zeros), which is pinned against the reference's packing."""
    rng = np.random.default_rng(7)
    counts = np.array([0, 300, 17, 256, 513, 1], dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    rows = int(offsets[-1])
    s = rng.integers(1, 255, (rows, 8), dtype=np.uint8)
    words = mx.gather_words(s, offsets, len(counts))
    m = 0
    for e in range(len(counts)):
        for row0 in range(int(offsets[e]), int(offsets[e + 1]), 256):
            n = min(256, int(offsets[e + 1]) - row0)
            np.testing.assert_array_equal(words[:, m * 256:(m + 1) * 256],
                                          mx.mx_pack_scales(_pad_rows(s[row0:row0 + n], 256)))
            m += 1
    assert not words[:, m * 256:].any()


def test_pack_weight_words_vs_pack():
    rng = np.random.default_rng(8)
    s = rng.integers(1, 255, (3, 512, 16), dtype=np.uint8)
    w = mx.pack_weight_words(s)
    for e in range(3):
        for nt in range(2):
            np.testing.assert_array_equal(w[e, nt], mx.mx_pack_scales(s[e, nt * 256:(nt + 1) * 256]))
    # fused gate/up rows: 64-row quarter q of B tile nt holds gate rows
    # nt*128 + 32q .. +31, then the matching up rows (+I)
    I = 256
    wg = mx.pack_weight_words(s, gate_up=I)
    for e in range(3):
        for nt in range(2):
            rows = [nt * 128 + 32 * (R // 64) + (R % 32) + (I if (R // 32) % 2 else 0) for R in range(256)]
            np.testing.assert_array_equal(wg[e, nt], mx.mx_pack_scales(s[e, rows]))


def test_moe_forward_mx_vs_per_token_bruteforce():
    """Per token, without permutation or grouped GEMMs: out[t] = bf16(sum_j
    w_j * bf16(deq(quant_mx(bf16(silu(g)*u))) . deq(W2[e_j])^T))."""
    from oracle import brute
    d = mx.make_mx_moe(T=20, H=256, I=128, E=6, k=3, skew=True, seed=9)
    r = mx.moe_forward_mx(d["x_q"], d["x_e8m0"], d["logits"], d["w13_q"], d["w13_e8m0"], d["w2_q"],
                          d["w2_e8m0"], 3, return_all=True)
    I = 128
    out = np.zeros((20, 256), dtype=np.float32)
    for t in range(20):
        sel, wts = brute.topk_bruteforce(d["logits"][t], 3)
        xt = mx.dequant_mx(d["x_q"][t:t + 1], d["x_e8m0"][t:t + 1])
        acc = np.float32(0) * np.zeros(256, np.float32)
        for j, e in enumerate(sel):
            z = (xt @ mx.dequant_mx(d["w13_q"][e], d["w13_e8m0"][e]).T).astype(np.float32)
            h = fp8.bf16_round(spec.silu_mul(z[:, :I], z[:, I:]))
            hq, hs = mx.quant_mx(h)
            y = fp8.bf16_round((mx.dequant_mx(hq, hs) @ mx.dequant_mx(d["w2_q"][e], d["w2_e8m0"][e]).T)
                               .astype(np.float32))
            acc = (acc + np.float32(wts[j]) * y[0]).astype(np.float32)
        out[t] = fp8.bf16_round(acc)
    np.testing.assert_array_equal(r["out"], out)
