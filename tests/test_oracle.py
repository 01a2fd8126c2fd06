"""Pins the CPU oracle (oracle/quant.py) before it is trusted as the checker.

The reference ships no tests or golden vectors for this path, so the oracle is
pinned by: known-answer blocks worked out by hand from the CUDA source,
an independent exact-arithmetic restatement (Python Fractions + a hand-written
round-to-nearest-even, no numpy casts) over random blocks including special
values, brute-force loops for the products, closed forms, and planted
mistakes that the acceptance tolerance must reject.
"""

from fractions import Fraction
import math

import numpy as np
import pytest
import torch

from oracle import quant as oq
from gdsllm_amd import synthetic as syn


# ---------------------------------------------------------------- exact rounding


def round_rne(x: Fraction, mant_bits: int, emin: int, emax: int) -> Fraction:
    """Round an exact rational to the nearest IEEE binary value with `mant_bits`
    significand bits (incl. the hidden bit), min normal exponent emin, max emax;
    ties to even; overflow -> +-inf (returned as float)."""
    if x == 0:
        return x
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)  # subnormals share the minimum exponent's ulp
    ulp = Fraction(2) ** (e - mant_bits + 1)
    q, r = divmod(a, ulp)
    q = int(q)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    v = q * ulp
    max_finite = (2 - Fraction(2) ** (1 - mant_bits)) * Fraction(2) ** emax
    if v > max_finite:
        return sign * math.inf
    return sign * v


def to_f16_bits(v) -> int:
    """Bits of an exactly representable fp16 value (Fraction / float / inf)."""
    return int(np.array([float(v)], dtype=np.float64).astype(np.float16).view(np.uint16)[0])


def f16(bits: int) -> Fraction:
    return Fraction(float(np.array([bits], dtype=np.uint16).view(np.float16)[0]))


def exact_q4_0(raw: np.ndarray) -> list:
    """Independent restatement of runtime/gguf_dequant.cu:84-107 with exact math."""
    out = []
    for blk in raw.reshape(-1, 18):
        d = f16(int(blk[0]) | (int(blk[1]) << 8))
        vals = [None] * 32
        for j in range(16):
            vals[j] = d * ((int(blk[2 + j]) & 15) - 8)
            vals[j + 16] = d * ((int(blk[2 + j]) >> 4) - 8)
        for j, v in enumerate(vals):
            # fp32 product is exact (11 x 4 bits), then one RNE to fp16
            r = round_rne(v, 11, -14, 15)
            neg_zero = v == 0 and (d < 0 or (d == 0 and str(float(d)).startswith("-"))) != (
                (((int(blk[2 + j % 16]) >> (4 * (j // 16))) & 15) - 8) < 0)
            out.append(0x8000 if (r == 0 and neg_zero) else to_f16_bits(r))
    return out


def _sign_bit(bits: int) -> bool:
    return bool(bits & 0x8000)


# ------------------------------------------------------------------ known answers


def test_q4_0_known_answer_block():
    """d = 1, qs[j] = (15-j) << 4 | j: element j = j-8 (low nibble), element
    j+16 = 7-j (high nibble) — the j / j+16 order of gguf_dequant.cu:105-106."""
    blk = np.zeros(18, dtype=np.uint8)
    blk[:2] = np.array([1.0], dtype=np.float16).view(np.uint8)
    for j in range(16):
        blk[2 + j] = ((15 - j) << 4) | j
    out = oq.dequant_q4_0(blk)
    assert out[:16].tolist() == [j - 8 for j in range(16)]
    assert out[16:].tolist() == [7 - j for j in range(16)]


def test_q4_0_signed_zeros():
    """d < 0 with q = 8 gives -0.0 (fp32 -0.5 * 0 = -0); d = +0 gives -0 for q < 8."""
    blk = np.zeros((2, 18), dtype=np.uint8)
    blk[0, :2] = np.array([-0.5], dtype=np.float16).view(np.uint8)
    blk[0, 2:] = 0x88
    blk[1, :2] = np.array([0.0], dtype=np.float16).view(np.uint8)
    blk[1, 2:] = 0x0F  # low nibble 15 (+7 * 0 = +0), high nibble 0 (-8 * 0 = -0)
    bits = oq.dequant_q4_0(blk).view(np.uint16)
    assert all(b == 0x8000 for b in bits[:32])
    assert all(b == 0x0000 for b in bits[32:48]) and all(b == 0x8000 for b in bits[48:])


def test_q8_0_known_answer_block():
    blk = np.zeros(34, dtype=np.uint8)
    blk[:2] = np.array([0.5], dtype=np.float16).view(np.uint8)
    q = np.array([-127, -128, -1, 0, 1, 127] + list(range(-13, 13)), dtype=np.int8)
    blk[2:] = q.view(np.uint8)
    assert oq.dequant_q8_0(blk).tolist() == [0.5 * v for v in q.tolist()]


def test_affine_nibble_order_lsb_first():
    """word 0x76543210 holds elements 0..7 = 0..7 (runtime/affine_q4_dequant.cu:50-58)."""
    w = np.array([0x76543210, 0xFEDCBA98], dtype=np.uint32)
    assert oq.unpack_affine_nibbles(w).tolist() == list(range(16))
    out = oq.dequant_affine_q4(w, np.array([1.0, 2.0], np.float16), np.array([0.0, -1.0], np.float16), 16, 8)
    assert out.tolist() == list(range(8)) + [2 * v - 1 for v in range(8, 16)]


def test_affine_group_is_flat_index():
    """Groups follow the flat element index, crossing row boundaries when
    in_dim is not a multiple of group_size (the reference's group_idx)."""
    w = np.full(6, 0x11111111, dtype=np.uint32)  # 48 nibbles of 1
    s = np.array([1.0, 2.0, 4.0], np.float16)
    out = oq.dequant_affine_q4(w, s, np.zeros(3, np.float16), 48, 16)
    assert out.tolist() == [1.0] * 16 + [2.0] * 16 + [4.0] * 16


# ----------------------------------------------------------- exact restatements


SPECIAL_D = [0.0, -0.0, 1.0, -1.0, 0.5, 6.0e-8, -5.96e-8, 3.0e-5, 65504.0, -65504.0, 7.1e3, 0.0123, 1e-3]


def _random_q4_blocks(n, seed):
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(n, 18), dtype=np.uint8)
    d = np.concatenate([np.array(SPECIAL_D, np.float16),
                        rng.uniform(-2, 2, n - len(SPECIAL_D)).astype(np.float16)])
    raw[:, :2] = d.view(np.uint8).reshape(n, 2)
    return raw


def test_q4_0_matches_exact_rounding():
    raw = _random_q4_blocks(64, 1)
    got = oq.dequant_q4_0(raw).view(np.uint16)
    for i, (g, blk) in enumerate(zip(got.reshape(-1, 32), raw)):
        d = f16(int(blk[0]) | (int(blk[1]) << 8))
        d_neg = bool(blk[1] & 0x80)
        for j in range(32):
            q = ((int(blk[2 + j % 16]) >> (4 * (j // 16))) & 15) - 8
            v = round_rne(d * q, 11, -14, 15)
            if v == 0:
                assert _sign_bit(int(g[j])) == (d_neg != (q < 0)) and int(g[j]) & 0x7FFF == 0, (i, j)
            else:
                assert int(g[j]) == to_f16_bits(v), (i, j)


def test_cpu_baseline_dequant_is_the_oracle_bit_for_bit():
    """The torch restatement timed as the CPU baseline dequantizes exactly as
    the oracle does (same bits, signed zeros and special scales included), and
    its GEMV is the fp32 product of those weights."""
    from oracle import cpu_baseline

    raw = _random_q4_blocks(256, 11)
    got = cpu_baseline.dequant_q4_0(torch.from_numpy(raw.copy())).numpy().view(np.uint16)
    assert np.array_equal(got, oq.dequant_q4_0(raw).view(np.uint16))
    M, K, B = 24, 256, 2
    w = syn.q4_0_weights(M, K, torch.Generator().manual_seed(12))
    x = syn.activations(B, K, torch.Generator().manual_seed(13))
    y = cpu_baseline.q4_0_gemv(w, x, M, K).numpy()
    deq = oq.dequant_q4_0(w.numpy()).reshape(M, K)
    rel, mx = oq.gemv_errors(y.astype(np.float64), oq.gemv(deq, x.numpy()), oq.row_norms(deq, x.numpy()))
    assert rel <= oq.GEMV_REL_L2 and mx <= oq.GEMV_MAX_NORM


def test_cpu_baseline_q8_0_affine_and_moe_loop_pinned():
    """The Q8_0 and affine-Q4 restatements timed as CPU baselines dequantize
    bit for bit as the oracle (special scales included); their GEMVs and the
    per-expert MoE decode loop stay within the GEMV tolerance of the oracle."""
    from oracle import cpu_baseline

    rng = np.random.default_rng(31)
    n = 64
    raw = rng.integers(0, 256, size=(n, 34), dtype=np.uint8)
    d = np.concatenate([np.array(SPECIAL_D, np.float16), rng.uniform(-0.01, 0.01, n - len(SPECIAL_D)).astype(np.float16)])
    raw[:, :2] = d.view(np.uint8).reshape(n, 2)
    got = cpu_baseline.dequant_q8_0(torch.from_numpy(raw.copy())).numpy().view(np.uint16)
    assert np.array_equal(got, oq.dequant_q8_0(raw).view(np.uint16))
    M, K, g = 40, 512, 64
    words, scales, biases = syn.affine_q4_weights([M, K], g, torch.Generator().manual_seed(32))
    want = oq.dequant_affine_q4(words.numpy(), scales.numpy(), biases.numpy(), M * K, g)
    got = cpu_baseline.dequant_affine_q4(words, scales, biases, g).numpy().reshape(-1)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    x = syn.activations(1, K, torch.Generator().manual_seed(33))
    w8 = syn.q8_0_weights(M, K, torch.Generator().manual_seed(34))
    deq8 = oq.dequant_q8_0(w8.numpy()).reshape(M, K)
    y8 = cpu_baseline.q8_0_gemv(w8, x, M, K).numpy()
    rel, mx = oq.gemv_errors(y8.astype(np.float64), oq.gemv(deq8, x.numpy()), oq.row_norms(deq8, x.numpy()))
    assert rel <= oq.GEMV_REL_L2 and mx <= oq.GEMV_MAX_NORM
    ya = cpu_baseline.affine_gemv(words, scales, biases, x, g).numpy()
    deqa = want.reshape(M, K)
    rel, mx = oq.gemv_errors(ya.astype(np.float64), oq.gemv(deqa, x.numpy()), oq.row_norms(deqa, x.numpy()))
    assert rel <= oq.GEMV_REL_L2 and mx <= oq.GEMV_MAX_NORM
    # the MoE decode loop over 6 experts, top 3, against oracle.moe_gather
    E, H, F, k = 6, 256, 128, 3
    gen = torch.Generator().manual_seed(35)
    pools = [syn.affine_q4_weights(sh, g, gen) for sh in ([E, F, H], [E, F, H], [E, H, F])]
    xm = syn.activations(1, H, gen)
    idx = [4, 0, 2]
    wts = torch.softmax(torch.randn(k, generator=gen), 0).to(torch.float16)

    def dq(pool, e, rows, cols):
        return oq.dequant_affine_q4(pool[0][e].numpy(), pool[1][e].numpy(), pool[2][e].numpy(), rows * cols,
                                    g).reshape(rows, cols)

    ref, _ = oq.moe_gather(xm.numpy(), lambda e: dq(pools[0], e, F, H), lambda e: dq(pools[1], e, F, H),
                           lambda e: dq(pools[2], e, H, F), idx, wts.numpy())
    got = cpu_baseline.moe_gather_decode(pools[0], pools[1], pools[2], xm, idx, wts, g).numpy().reshape(-1)
    assert float(np.linalg.norm(got - ref) / np.linalg.norm(ref)) <= oq.GEMV_REL_L2


def test_q8_0_matches_exact_rounding():
    rng = np.random.default_rng(2)
    n = 64
    raw = rng.integers(0, 256, size=(n, 34), dtype=np.uint8)
    d = np.concatenate([np.array(SPECIAL_D, np.float16), rng.uniform(-0.01, 0.01, n - len(SPECIAL_D)).astype(np.float16)])
    raw[:, :2] = d.view(np.uint8).reshape(n, 2)
    got = oq.dequant_q8_0(raw).view(np.uint16)
    for g, blk in zip(got.reshape(-1, 32), raw):
        dd = f16(int(blk[0]) | (int(blk[1]) << 8))
        d_neg = bool(blk[1] & 0x80)
        for j in range(32):
            q = int(np.int8(np.uint8(blk[2 + j])))
            v = round_rne(dd * q, 11, -14, 15)
            if v == 0:
                assert _sign_bit(int(g[j])) == (d_neg != (q < 0)) and int(g[j]) & 0x7FFF == 0
            else:
                assert int(g[j]) == to_f16_bits(v)


def test_affine_matches_exact_double_rounding():
    """nib*s + b rounded once to fp32, then once to fp16 — not a single rounding."""
    rng = np.random.default_rng(3)
    groups, g = 40, 16
    w = rng.integers(0, 2**32, size=groups * g // 8, dtype=np.uint64).astype(np.uint32)
    s = np.concatenate([np.array([1.0, -2.0, 6.0e-8, 65504.0, 0.0], np.float16),
                        rng.uniform(0.005, 0.02, groups - 5).astype(np.float16)])
    b = np.concatenate([np.array([1e-7, 3.0, -65504.0, 1.0, -0.0], np.float16),
                        (rng.normal(0, 0.05, groups - 5)).astype(np.float16)])
    got = oq.dequant_affine_q4(w, s, b, groups * g, g).view(np.uint16)
    nib = oq.unpack_affine_nibbles(w)
    for i in range(groups * g):
        G = i // g
        exact = int(nib[i]) * Fraction(float(s[G])) + Fraction(float(b[G]))
        v32 = round_rne(exact, 24, -126, 127)
        v = round_rne(Fraction(v32) if not isinstance(v32, float) else v32, 11, -14, 15) if not isinstance(v32, float) else v32
        if v == 0:
            continue  # sign of an exact zero sum: fp32 rules (x + -x = +0) checked below
        assert int(got[i]) == to_f16_bits(v), i
    # exact zero: 0*s + (-0) = +0 in round-to-nearest (fp32 add of +0 and -0)
    z = oq.dequant_affine_q4(np.zeros(1, np.uint32), np.array([1.0], np.float16), np.array([-0.0], np.float16), 8, 8)
    assert z.view(np.uint16).tolist() == [0] * 8


# ------------------------------------------------------------------ products


def test_gemv_brute_force():
    rng = np.random.default_rng(4)
    M, K, B = 5, 64, 3
    raw = syn.q4_0_weights(M, K, torch.Generator().manual_seed(4)).numpy()
    w = oq.dequant_q4_0(raw).reshape(M, K)
    x = rng.normal(size=(B, K)).astype(np.float16)
    y = oq.gemv(w, x)
    for b in range(B):
        for r in range(M):
            ref = math.fsum(float(w[r, k]) * float(x[b, k]) for k in range(K))
            assert abs(y[b, r] - ref) <= 1e-12 * max(1.0, abs(ref))
    norms = oq.row_norms(w, x)
    for b in range(B):
        for r in range(M):
            assert abs(norms[b, r] - math.sqrt(sum((float(w[r, k]) * float(x[b, k])) ** 2 for k in range(K)))) < 1e-9


def test_gemv_ieee_special_values():
    """IEEE results of the reference's fp32 loop: a nonzero weight times inf
    is +-inf, a zero weight times inf is NaN, +inf and -inf terms give NaN, NaN
    propagates; finite inputs give gemv's value."""
    inf, nan = np.inf, np.nan
    w = np.array([[1.0, 0.5, 0.0], [0.0, 1.0, 1.0], [-2.0, 1.0, 0.0], [1.0, -1.0, 0.0]], np.float16)
    x = np.array([[inf, 1.0, 2.0], [inf, inf, 1.0], [nan, 1.0, 1.0]], np.float16)
    y = oq.gemv_ieee(w, x)
    assert y[0, 0] == inf and np.isnan(y[0, 1]) and y[0, 2] == -inf and y[0, 3] == inf
    assert y[1, 0] == inf and np.isnan(y[1, 1]) and np.isnan(y[1, 2]) and np.isnan(y[1, 3])
    assert np.isnan(y[2]).all()
    rng = np.random.default_rng(21)
    wf = rng.normal(size=(7, 96)).astype(np.float16)
    xf = rng.normal(size=(2, 96)).astype(np.float16)
    ref = np.array([[math.fsum(float(a) * float(b) for a, b in zip(wr, xr)) for wr in wf] for xr in xf])
    assert np.allclose(oq.gemv_ieee(wf, xf, rows_per_chunk=3), ref, rtol=1e-12, atol=1e-12)


def test_gemv_closed_forms():
    M, K = 8, 256
    raw = syn.q4_0_weights(M, K, torch.Generator().manual_seed(5)).numpy().reshape(-1, 18).copy()
    raw[:, 2:] = 0x88
    w = oq.dequant_q4_0(raw).reshape(M, K)
    x = np.random.default_rng(5).normal(size=(1, K)).astype(np.float16)
    assert np.all(oq.gemv(w, x) == 0)
    raw2 = syn.q4_0_weights(M, K, torch.Generator().manual_seed(6)).numpy()
    w2 = oq.dequant_q4_0(raw2).reshape(M, K)
    e = np.zeros((1, K), np.float16)
    e[0, 37] = 1
    assert np.array_equal(oq.gemv(w2, e)[0], w2[:, 37].astype(np.float64))


def _fp32_kernel_model(raw, M, K, x, *, swap_nibbles=False, drop_offset=False, shift_scale=False):
    """fp32-accumulating model of a fused GEMV, optionally with a planted mistake."""
    b = raw.reshape(-1, 18)
    d = b[:, :2].copy().view(np.float16)[:, 0].astype(np.float32)
    if shift_scale:
        d = np.roll(d, 1)
    qs = b[:, 2:]
    lo, hi = (qs & 15).astype(np.float32), (qs >> 4).astype(np.float32)
    if swap_nibbles:
        lo, hi = hi, lo
    off = 0.0 if drop_offset else 8.0
    w = np.concatenate([(lo - off), (hi - off)], axis=1) * d[:, None]
    w = w.reshape(M, K).astype(np.float32)
    return (x.astype(np.float32) @ w.T).astype(np.float16)


@pytest.mark.parametrize("mistake", ["swap_nibbles", "drop_offset", "shift_scale"])
def test_tolerance_rejects_planted_mistakes(mistake):
    """A correct fp32 model passes the acceptance test; each plausible slip fails it."""
    M, K = 64, 1024
    raw = syn.q4_0_weights(M, K, torch.Generator().manual_seed(7)).numpy()
    x = np.random.default_rng(7).normal(size=(1, K)).astype(np.float16)
    w = oq.dequant_q4_0(raw).reshape(M, K)
    ref, norms = oq.gemv(w, x), oq.row_norms(w, x)
    good = oq.gemv_errors(_fp32_kernel_model(raw, M, K, x), ref, norms)
    assert good[0] <= oq.GEMV_REL_L2 and good[1] <= oq.GEMV_MAX_NORM
    bad = oq.gemv_errors(_fp32_kernel_model(raw, M, K, x, **{mistake: True}), ref, norms)
    assert bad[0] > oq.GEMV_REL_L2 or bad[1] > oq.GEMV_MAX_NORM


def test_row_bound_charges_only_beyond_one_output_ulp():
    """Affine rows against a positive x have |y| >> ||w*x||: the correctly rounded
    fp16 result passes the per-row bound, and so does anything within one ulp,
    but 3 ulps off, a dropped group or a lost bias fails it."""
    M, K, g = 128, 4096, 64
    w, s, b = syn.affine_q4_weights([M, K], g, torch.Generator().manual_seed(11))
    wq = oq.dequant_affine_q4(w.numpy().view(np.uint32), s.numpy(), b.numpy(), M * K, g).reshape(M, K)
    x = np.abs(np.random.default_rng(11).normal(size=(1, K))).astype(np.float16)
    ref, norms = oq.gemv(wq, x), oq.row_norms(wq, x)
    assert np.max(np.abs(ref) / norms) > 30  # the regime the allowance is for
    y16 = ref.astype(np.float16)
    assert np.max(np.abs(y16 - ref) / norms) > oq.GEMV_MAX_NORM  # the plain bound would reject it
    assert oq.gemv_errors(y16, ref, norms)[1] == 0.0
    ulp = oq.fp16_ulp(ref)
    assert oq.gemv_errors(ref + 0.99 * ulp, ref, norms)[1] == 0.0
    assert oq.gemv_errors(ref + 3 * ulp, ref, norms)[1] > oq.GEMV_MAX_NORM
    dropped = oq.gemv(np.concatenate([wq[:, : K - g], np.zeros((M, g), np.float16)], axis=1), x)
    assert oq.gemv_errors(dropped.astype(np.float16), ref, norms)[1] > oq.GEMV_MAX_NORM
    wq_nobias = oq.dequant_affine_q4(w.numpy().view(np.uint32), s.numpy(), np.zeros_like(b.numpy()), M * K, g)
    nobias = oq.gemv(wq_nobias.reshape(M, K), x).astype(np.float16)
    assert oq.gemv_errors(nobias, ref, norms)[1] > oq.GEMV_MAX_NORM


def test_moe_gather_composition():
    """top_k = 1 with weight 1 equals down . fp16(fp16(silu(fp16(gate.x))) * fp16(up.x));
    the result is linear in the routing weights; unknown experts add nothing."""
    rng = np.random.default_rng(8)
    H, F = 64, 32
    mats = {e: [rng.normal(0, 0.1, size=s).astype(np.float16) for s in ((F, H), (F, H), (H, F))] for e in range(3)}
    gate = lambda e: mats[e][0] if e in mats else None  # noqa: E731
    up = lambda e: mats[e][1] if e in mats else None  # noqa: E731
    down = lambda e: mats[e][2] if e in mats else None  # noqa: E731
    x = rng.normal(size=H).astype(np.float16)
    y1, hs = oq.moe_gather(x, gate, up, down, [2], [1.0])
    g = (mats[2][0].astype(np.float64) @ x.astype(np.float64)).astype(np.float16)
    u = (mats[2][1].astype(np.float64) @ x.astype(np.float64)).astype(np.float16)
    gf = g.astype(np.float32)
    sg = (gf / (1 + np.exp(-gf))).astype(np.float16)
    h = (sg.astype(np.float32) * u.astype(np.float32)).astype(np.float16)
    assert np.array_equal(hs[0], h)
    assert np.allclose(y1, mats[2][2].astype(np.float64) @ h.astype(np.float64), rtol=0, atol=1e-12)
    ya, _ = oq.moe_gather(x, gate, up, down, [0, 1], [0.25, 0.75])
    y0, _ = oq.moe_gather(x, gate, up, down, [0], [1.0])
    yb, _ = oq.moe_gather(x, gate, up, down, [1], [1.0])
    assert np.allclose(ya, 0.25 * y0 + 0.75 * yb, rtol=1e-12, atol=1e-12)
    yc, _ = oq.moe_gather(x, gate, up, down, [0, 7, 1], [0.25, 0.5, 0.75])
    assert np.allclose(yc, ya, rtol=0, atol=0)


def test_moe_prefill_matches_token_by_token_loop():
    """The prefill oracle groups tokens by expert per slot; an independent loop
    over tokens (one token at a time, slots in order, the same fp16 steps
    written out by hand with Fraction-free float64 products) must give the same
    bits, and one token with one slot of weight 1 equals the decode oracle's h
    and down product rounded to fp16."""
    rng = np.random.default_rng(11)
    H, F, E, T, k = 64, 32, 5, 9, 3
    mats = {e: [rng.normal(0, 0.1, size=s).astype(np.float16) for s in ((F, H), (F, H), (H, F))] for e in range(E)}
    gate = lambda e: mats[e][0] if e in mats else None  # noqa: E731
    up = lambda e: mats[e][1] if e in mats else None  # noqa: E731
    down = lambda e: mats[e][2] if e in mats else None  # noqa: E731
    x = rng.normal(size=(T, H)).astype(np.float16)
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    idx[2, 1] = -1   # an index outside the pool contributes nothing
    idx[5, 0] = E
    w = (rng.random((T, k)) / k).astype(np.float16)
    out, inter = oq.moe_prefill(x, gate, up, down, idx, w)
    for t in range(T):
        acc = np.float16(0)
        for j in range(k):
            e = int(idx[t, j])
            if e not in mats:
                assert (t, j) not in inter
                continue
            xt = x[t].astype(np.float64)
            g = (mats[e][0].astype(np.float64) @ xt).astype(np.float16)
            u = (mats[e][1].astype(np.float64) @ xt).astype(np.float16)
            gf = g.astype(np.float32)
            h = ((gf / (np.float32(1) + np.exp(-gf))).astype(np.float16).astype(np.float32) * u.astype(np.float32)).astype(np.float16)
            d = (mats[e][2].astype(np.float64) @ h.astype(np.float64)).astype(np.float16)
            assert np.array_equal(inter[(t, j)][0], h) and np.array_equal(inter[(t, j)][1], d)
            acc = (np.float32(acc) + (np.float32(w[t, j]) * d.astype(np.float32)).astype(np.float16).astype(np.float32)).astype(np.float16)
        assert np.array_equal(out[t].view(np.uint16), np.asarray(acc, dtype=np.float16).view(np.uint16)), t
    # one slot, weight 1: the decode oracle's float64 sum rounds to the same value
    y1, hs = oq.moe_gather(x[0], gate, up, down, idx[0, :1], [1.0])
    o1, _ = oq.moe_prefill(x[:1], gate, up, down, idx[:1, :1], np.ones((1, 1), np.float16))
    assert np.array_equal(o1[0], y1.astype(np.float16))
    # the combine alone, replayed from the intermediates and positions
    pos = np.full((T, k), -1)
    rows = []
    for (t, j), (_h, d) in sorted(inter.items()):
        pos[t, j] = len(rows)
        rows.append(d)
    assert np.array_equal(oq.moe_prefill_combine(np.stack(rows), pos, w).view(np.uint16), out.view(np.uint16))
    # a planted mistake (slots summed in reverse order) changes some bits
    rev = oq.moe_prefill_combine(np.stack(rows), pos[:, ::-1].copy(), w[:, ::-1].copy())
    assert not np.array_equal(rev.view(np.uint16), out.view(np.uint16))


def test_affine_double_rounding_follows_reference():
    """Cases where rounding nib*s+b straight to fp16 differs from the reference's
    fp32-then-fp16 exist; the oracle gives the reference's value (checked with
    the exact-arithmetic rounding above, independent of numpy casts)."""
    from helpers import double_rounding_cases

    nib, s, b = double_rounding_cases(32, 9)
    for i in range(len(nib)):
        exact = int(nib[i]) * Fraction(float(s[i])) + Fraction(float(b[i]))
        direct = round_rne(exact, 11, -14, 15)
        twice = round_rne(round_rne(exact, 24, -126, 127), 11, -14, 15)
        assert direct != twice
        out = oq.dequant_affine_q4(np.array([nib[i]], np.uint32), s[i:i + 1], b[i:i + 1], 8, 8)
        assert out.view(np.uint16)[0] == to_f16_bits(twice)


# ------------------------------------------------------------- MoE routing


def _topk_lexsort(v: np.ndarray, k: int) -> np.ndarray:
    """Independent restatement of the pick order with np.lexsort: NaN first,
    then value descending (-0 == +0), then index ascending."""
    x = v.astype(np.float64)
    nan = np.isnan(x)
    val = np.where(nan, 0.0, -x) + 0.0  # + 0.0 turns -0 into +0
    order = np.lexsort((np.arange(v.size), val, ~nan))
    return order[:k]


@pytest.mark.parametrize("seed", range(6))
def test_route_topk_order_matches_lexsort(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(8, 300))
    k = int(rng.integers(1, min(E, 64) + 1))
    # few distinct values: many ties; plus specials
    v = rng.integers(-4, 5, size=(3, E)).astype(np.float16) * np.float16(0.5)
    v[0, rng.integers(0, E, 3)] = np.float16(np.nan)
    v[1, rng.integers(0, E, 3)] = np.float16(-np.inf)
    v[2, rng.integers(0, E, 3)] = np.float16(-0.0)
    idx, w = oq.route_topk(v, k)
    for t in range(3):
        assert list(idx[t]) == list(_topk_lexsort(v[t], k))


def test_route_topk_softmax_closed_forms():
    # k = 1: weight exactly 1; two equal logits: 0.5 each; exp(0) / (1 + e^-1)
    idx, w = oq.route_topk(np.array([[0.25, 3.0, -1.0]], np.float16), 1)
    assert idx[0, 0] == 1 and w[0, 0] == np.float16(1.0)
    idx, w = oq.route_topk(np.array([[2.0, -5.0, 2.0]], np.float16), 2)
    assert list(idx[0]) == [0, 2] and list(w[0]) == [np.float16(0.5)] * 2
    idx, w = oq.route_topk(np.array([[1.0, 0.0]], np.float16), 2)
    e = math.exp(-1.0)
    assert w[0, 0] == np.float16(1.0 / (1.0 + e)) and w[0, 1] == np.float16(e / (1.0 + e))
    # weights of random rows sum to 1 within k half-ulps of 1 and do not increase
    rng = np.random.default_rng(7)
    idx, w = oq.route_topk(rng.standard_normal((4, 512)).astype(np.float16), 10)
    ws = w.astype(np.float64)
    assert np.all(np.abs(ws.sum(axis=1) - 1.0) <= 10 * 2.0 ** -11)
    assert np.all(np.diff(ws, axis=1) <= 0)
    # a planted mistake (picking the smallest) fails the lexsort check
    v = rng.standard_normal(50).astype(np.float16)
    assert list(np.argsort(v)[:5]) != list(_topk_lexsort(v, 5))


def test_moe_combine_closed_forms():
    eo = np.array([[1.0, -2.0, np.inf, np.nan, -60000.0, 3.0]], np.float16)
    so = np.array([[2.0, 4.0, 1.0, 1.0, -60000.0, -6.0]], np.float16)
    # g = 0: sigmoid = 0.5 exactly, so s = so / 2 exactly
    r = oq.moe_combine(eo, so, [0.0])
    assert list(r[0, :3]) == [np.float16(2.0), np.float16(0.0), np.float16(65504.0)]
    assert np.isnan(r[0, 3]) and r[0, 4] == np.float16(-65504.0) and r[0, 5] == np.float16(0.0)
    # g very negative: sigmoid rounds to 0 in fp16 -> r = eo (finite entries)
    r = oq.moe_combine(np.array([[1.5, -7.0]], np.float16), np.array([[100.0, 100.0]], np.float16), [-30.0])
    assert list(r[0]) == [np.float16(1.5), np.float16(-7.0)]
    # g large: sigmoid = 1 -> r = fp16(eo + so)
    r = oq.moe_combine(np.array([[1.0, 1024.0]], np.float16), np.array([[2.0, 0.5]], np.float16), [20.0])
    assert list(r[0]) == [np.float16(3.0), np.float16(1024.0)]


def test_silu_fp16_against_torch_over_every_fp16():
    """silu_fp16 (the fp16 F.silu step of qwen_moe.py:471) against torch's own
    CPU F.silu on all 65,536 fp16 inputs: bit-equal except 3 inputs at one ulp
    (torch's vectorized exp rounds differently there); +-inf and NaN behave
    alike.  A planted mistake (sigmoid without the factor x) fails."""
    torch = pytest.importorskip("torch")
    allh = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    with np.errstate(all="ignore"):
        got = oq.silu_fp16(allh)
        bad = (np.float32(1.0) / (np.float32(1.0) + np.exp(-allh.astype(np.float32)))).astype(np.float16)
    want = torch.nn.functional.silu(torch.from_numpy(allh.copy())).numpy()
    same = (got.view(np.uint16) == want.view(np.uint16)) | (np.isnan(got) & np.isnan(want))
    assert (~same).sum() <= 3
    diff = np.abs(got[~same].astype(np.float64) - want[~same].astype(np.float64))
    assert np.all(diff <= oq.fp16_ulp(want[~same].astype(np.float64)))
    planted = (bad.view(np.uint16) == want.view(np.uint16)) | (np.isnan(bad) & np.isnan(want))
    assert (~planted).sum() > 10000


# ------------------------------------------------------- per-column int8 weights


def test_int8_matches_exact_rounding():
    """Every q in [-128, 127] against special and random column scales, each
    product rounded once with exact arithmetic; the sign of zero follows
    IEEE (0 * negative scale = -0)."""
    rng = np.random.default_rng(3)
    scales = np.concatenate([np.array(SPECIAL_D, np.float16), rng.uniform(-0.01, 0.01, 24).astype(np.float16)])
    q = np.arange(-128, 128, dtype=np.int16).astype(np.int8)[:, None].repeat(scales.size, axis=1)
    got = oq.dequant_int8(q, scales.reshape(1, -1)).view(np.uint16)
    for c, s in enumerate(scales):
        sv = Fraction(float(s)) if np.isfinite(s) else None
        s_neg = bool(np.array([s], np.float16).view(np.uint16)[0] & 0x8000)
        for r in range(256):
            qv = int(q[r, c])
            g = int(got[r, c])
            if sv is None:
                continue
            v = round_rne(sv * qv, 11, -14, 15)
            if v == 0:
                assert _sign_bit(g) == (s_neg != (qv < 0)) and g & 0x7FFF == 0, (qv, s)
            else:
                assert g == to_f16_bits(v), (qv, s)


def test_int8_scale_is_per_column():
    """q = 1 everywhere returns each column's scale in every row: a scale
    broadcast along rows instead of columns fails."""
    scale = np.arange(1, 9, dtype=np.float16).reshape(1, 8) * np.float16(0.125)
    out = oq.dequant_int8(np.ones((3, 8), np.int8), scale)
    assert np.array_equal(out, np.repeat(scale, 3, axis=0))


def test_int8_quantizer_round_trip():
    """The restated converter quantizer (tools/convert_weights.py:55-83) and the
    dequant invert each other to within half a column scale; the extreme of
    each column maps to +-127."""
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((64, 96)) * rng.uniform(0.01, 1.0, 96)).astype(np.float16)
    q, s = oq.quantize_int8(w)
    assert q.dtype == np.int8 and s.shape == (1, 96)
    back = oq.dequant_int8(q, s).astype(np.float64)
    err = np.abs(back - w.astype(np.float64))
    # rounding to q (half the exact scale), the fp16 rounding of the stored
    # scale (times |q|), and the fp16 rounding of the dequantized product
    s_exact = np.abs(w.astype(np.float64)).max(axis=0, keepdims=True) / 127.0
    bound = 0.5 * s_exact + np.abs(q) * np.abs(s.astype(np.float64) - s_exact) + np.abs(back) * 2.0 ** -11 + 1e-12
    assert np.all(err <= bound * (1 + 1e-6))
    assert np.all(np.abs(q).max(axis=0) == 127)


def test_int8_gemv_brute_force():
    """oq.gemv over the int8 dequant equals a plain loop over exact products."""
    rng = np.random.default_rng(5)
    q = rng.integers(-128, 128, (5, 48)).astype(np.int8)
    s = rng.uniform(0.001, 0.004, (1, 48)).astype(np.float16)
    x = rng.standard_normal((2, 48)).astype(np.float16)
    w = oq.dequant_int8(q, s)
    want = [[sum(float(w[r, k]) * float(x[b, k]) for k in range(48)) for r in range(5)] for b in range(2)]
    assert np.allclose(oq.gemv(w, x), np.array(want), rtol=1e-12, atol=1e-12)
