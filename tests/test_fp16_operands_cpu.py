"""CPU emulation of the fp16 operands of the matrix-core decode kernels (numpy).

The f16 and int4 decode kernels (decode_mfma.hip, decode_mfma_int4.hip) feed two values to
fp16 MFMA operands that the reference keeps in fp32/double (attention_ref.c:50-79,
three_bit_runtime_modules.c:175-250):

  * q' = clip(q) * scale * log2(e), split into fp16 hi + lo (both kernels);
  * P' = p * (V scale), rounded once to fp16 (int4 kernel), where the lazy running max lets
    p = exp2(score - m_run) reach 2^thr (thr = 8 unless lowered).

These tests restate the conversions in numpy float16 and check (1) that the plain conversion
does fail where the GPU tests put the data (q' beyond 65504, P' beyond 65504, q' in the
subnormal range), and (2) that the rules the kernels apply keep every operand finite and
precise over the whole float range:

  * q' of one head is shifted by 2^e (e = 0 when max|q'| lies in [2^-4, 2^15), else max|q'|
    * 2^e lands in [2^14, 2^15)), split, and the score is multiplied by 2^-e;
  * a tile pair whose largest V scale s satisfies s >= 2^(16 - thr) lowers thr to
    15 - floor(log2 s) before P' is formed.
"""
import numpy as np

F16_MAX = 65504.0


def qnorm_shift(amax: float) -> int:
    """The kernels' shift rule (kv_common.h qnorm_shift)."""
    if not (amax > 0.0) or not np.isfinite(amax) or (0.0625 <= amax < 32768.0):
        return 0
    _, x = np.frexp(np.float32(amax))  # amax in [2^(x-1), 2^x)
    return int(min(max(15 - int(x), -100), 100))


def split(qv: np.ndarray):
    hi = qv.astype(np.float16)
    lo = (qv - hi.astype(np.float32)).astype(np.float16)
    return hi, lo


def scores_via_operands(q32: np.ndarray, k16: np.ndarray, e: int) -> np.ndarray:
    """Scores as the MFMAs form them: exact fp16 x fp16 products, the hi and lo chains
    summed, then the 2^-e factor (float64 stands in for the fp32 accumulators)."""
    qs = (q32.astype(np.float64) * 2.0 ** e).astype(np.float32)
    hi, lo = split(qs)
    k = k16.astype(np.float64)
    s = k @ hi.astype(np.float64) + k @ lo.astype(np.float64)
    return s * 2.0 ** (-e)


def _q_prime(rng, D, std, scale):
    q = (rng.standard_normal(D) * std).astype(np.float32)
    th = np.float32(4.5) * np.float32(q.astype(np.float64).std())
    return (np.clip(q, -th, th) * np.float32(scale * np.log2(np.e))).astype(np.float32)


def test_plain_split_overflows_for_huge_queries():
    """Mode P, std(q) = 2e5, caller scale 1.0: the plain hi of q' is infinite, so the
    score MFMA would return inf/NaN."""
    rng = np.random.default_rng(1)
    qp = _q_prime(rng, 64, 2e5, 1.0)
    with np.errstate(over="ignore", invalid="ignore"):
        hi, _ = split(qp)
    assert np.isinf(hi.astype(np.float32)).any()
    e = qnorm_shift(float(np.abs(qp).max()))
    assert e < 0
    hi, lo = split((qp.astype(np.float64) * 2.0 ** e).astype(np.float32))
    assert np.isfinite(hi.astype(np.float32)).all() and np.abs(hi.astype(np.float32)).max() < F16_MAX


def test_shifted_scores_keep_fp32_precision():
    """Over q' magnitudes from 1e-30 to 1e30 the shifted split gives scores within 2^-20 of
    sum |q' k| of the exact (float64) scores; the plain split fails at both ends."""
    rng = np.random.default_rng(2)
    D = 128
    k16 = (rng.standard_normal((64, D)) * 3.0).astype(np.float16)
    for mag in (1e-30, 1e-12, 1e-6, 1e-4, 1e-2, 0.1, 1.0, 100.0, 3e4, 1e5, 1e9, 1e30):
        qp = (rng.standard_normal(D) * mag).astype(np.float32)
        exact = k16.astype(np.float64) @ qp.astype(np.float64)
        bound = np.abs(k16.astype(np.float64)) @ np.abs(qp.astype(np.float64))
        e = qnorm_shift(float(np.abs(qp).max()))
        got = scores_via_operands(qp, k16, e)
        assert np.all(np.abs(got - exact) <= 2.0 ** -20 * bound), mag
        with np.errstate(over="ignore", invalid="ignore"):
            plain = scores_via_operands(qp, k16, 0)
        ok_plain = np.isfinite(plain).all() and np.all(np.abs(plain - exact) <= 2.0 ** -20 * bound)
        if mag <= 1e-4 or mag >= 1e5:
            assert not ok_plain, mag  # the plain split fails at both ends
        if e == 0:
            assert ok_plain, mag


def test_shift_rule_range():
    for amax in np.geomspace(1e-38, 3e38, 4000):
        e = qnorm_shift(float(amax))
        y = float(amax) * 2.0 ** e
        if 0.0625 <= amax < 32768.0:
            assert e == 0
        elif 2.0 ** -100 * 2 ** 14 <= amax <= 2.0 ** 100 * 2 ** 15:
            assert 2.0 ** 14 <= y < 2.0 ** 15, amax
        # 2^e and 2^-e are normal floats
        assert -126 <= e <= 127 and -126 <= -e <= 127
    assert qnorm_shift(0.0) == 0 and qnorm_shift(float("inf")) == 0 and qnorm_shift(float("nan")) == 0


def test_p_times_vscale_overflows_without_the_bound():
    """p up to 2^8 times a V scale of 790 (|v| ~ 6e3) is ~2e5: fp16 overflows."""
    with np.errstate(over="ignore"):
        pq = (np.float32(2.0 ** 7.9) * np.float32(790.0)).astype(np.float16)
    assert np.isinf(pq)


def test_vscale_bound_keeps_p_prime_finite():
    """For every fp16 V scale s and every p <= 2^thr once thr is lowered by the rule, P' =
    fp16(p * s) <= 65504; without lowering, s >= 2^(16 - thr) can overflow."""
    scales = np.arange(0x0001, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    for thr0 in (8, 5, 0):
        bound = 2.0 ** (16 - thr0)
        for s in scales[::97].tolist() + [F16_MAX, bound, bound * (1 - 2 ** -11)]:
            s = float(np.float16(s))
            if not np.isfinite(s):
                continue
            thr = thr0
            if s >= 2.0 ** (16 - thr):
                x = int(np.floor(np.log2(s)))
                thr = min(thr, 15 - x)
            # v_exp_f32 is within 1 ulp of 2^thr
            p = np.float32(2.0 ** thr) * np.float32(1 + 2 ** -23)
            with np.errstate(over="ignore"):
                pq = np.float16(np.float32(p) * np.float32(s))
            assert np.isfinite(pq) and float(pq) <= F16_MAX, (thr0, s)
            assert thr >= 0
