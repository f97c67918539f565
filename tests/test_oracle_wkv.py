"""Pins the CPU oracle (oracle/wkv_oracle.c) before anything is compared with it.

The reference ships no golden vectors for the WKV path (its monkey-patch
fixtures are absent and its WKV unit tests assert no values), so the oracle is
pinned by what the mathematics fixes:
  * closed forms of the decay and of recurrence special cases that reduce to
    textbook matrix algebra (diagonal decay, rank-1 update, the classic delta
    rule, the one-token zero-state output);
  * a float64 brute force on tiny inputs;
  * exact rational arithmetic for the fp16 primitives;
  * size-independent invariants (prefill == repeated decode, dither phase
    bookkeeping).
One test plants a mistake (a dropped sa*b term) in a float64 restatement and
shows that the delta-rule closed form rejects it.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as orc
from tests.wkv_inputs import make_state, make_wkv_inputs

E_HALF = math.exp(-0.5)


def decay64(w):
    return np.exp(-E_HALF / (1.0 + np.exp(-np.asarray(w, dtype=np.float64))))


# ------------------------------------------------------------------ decay


def test_decay_closed_forms():
    assert orc.decay(0.0) == pytest.approx(math.exp(-E_HALF / 2), rel=2e-7)
    assert orc.decay(float("inf")) == pytest.approx(math.exp(-E_HALF), rel=2e-7)
    assert orc.decay(float("-inf")) == 1.0
    assert math.isnan(orc.decay(float("nan")))
    # sigmoid(w) + sigmoid(-w) = 1  =>  d(w) * d(-w) = exp(-e^{-1/2})
    for w in (0.3, 1.7, 5.0):
        assert orc.decay(w) * orc.decay(-w) == pytest.approx(math.exp(-E_HALF), rel=5e-7)


def test_decay_every_fp16_input():
    ws = np.arange(65536, dtype=np.uint16).view(np.float16)
    ws = ws[np.isfinite(ws)]
    got = np.array([orc.decay(float(w)) for w in ws], dtype=np.float64)
    rel = np.abs(got / decay64(ws.astype(np.float64)) - 1.0)
    assert rel.max() < 2.5e-7


def test_exp2_accuracy_and_range():
    xs = np.linspace(-125.0, 127.0, 20001, dtype=np.float32)
    got = np.array([orc.exp2(float(x)) for x in xs], dtype=np.float64)
    assert np.max(np.abs(got / np.exp2(xs.astype(np.float64)) - 1)) < 1.2e-7
    assert orc.exp2(0.0) == 1.0 and orc.exp2(1.0) == 2.0 and orc.exp2(-3.0) == 0.125
    assert orc.exp2(200.0) == float("inf") and orc.exp2(-200.0) == 0.0


def test_rotator_known_answers():
    assert orc.rotator(0) == 0.0
    # 2654435769 wraps to int32 -1640531527
    assert orc.rotator(1) == np.float32(-1640531527.0) * np.float32(2.0 ** -41)
    # 2 * 2654435769 mod 2^32 = 1013904242
    assert orc.rotator(2) == np.float32(1013904242.0) * np.float32(2.0 ** -41)
    assert orc.rotator(-1) == np.float32(1640531527.0) * np.float32(2.0 ** -41)


def test_w_delta_known_answer():
    want = np.float16(math.exp(-E_HALF / 2) - 1.0)
    assert orc.w_delta(0.0, 0) == want.view(np.uint16)


# ------------------------------------------------------------------ fp16 primitives


def _f16_exact(fr):
    """Round a Fraction to binary16, nearest-even, with exact rational arithmetic."""
    if fr == 0:
        return np.float16(0.0)
    sign = -1 if fr < 0 else 1
    x = abs(fr)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    ulp = Fraction(2) ** (max(e, -14) - 10)
    q = x / ulp
    n = q.numerator // q.denominator
    rem = q - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = n * ulp
    if v >= 65536:
        return np.float16(sign * np.inf)
    return np.float16(sign * float(v))


def _rand_halves(rng, n):
    bits = rng.integers(0, 65536, size=n, dtype=np.uint16)
    h = bits.view(np.float16)
    return h[np.isfinite(h)]


def test_fp16_primitives_exact():
    rng = np.random.default_rng(0)
    a, b, c = (_rand_halves(rng, 6000)[:4000] for _ in range(3))
    # also a band of magnitudes where products and addends interact (ties, cancellation)
    near = (rng.standard_normal((3, 3000)) * 4).astype(np.float16)
    a, b, c = (np.concatenate([x, y]) for x, y in zip((a, b, c), near))
    for x, y, z in zip(a, b, c):
        fx, fy, fz = (Fraction(float(t)) for t in (x, y, z))
        want = _f16_exact(fx * fy + fz)
        got = np.uint16(orc.fma16_bits(x.view(np.uint16), y.view(np.uint16), z.view(np.uint16))).view(np.float16)
        if np.isinf(want):
            assert np.isinf(got) and np.sign(got) == np.sign(want)
        else:
            assert got == want, (x, y, z, got, want)
        assert np.uint16(orc.add16_bits(x.view(np.uint16), z.view(np.uint16))).view(np.float16) == _f16_exact(fx + fz) or np.isinf(_f16_exact(fx + fz))
        assert np.uint16(orc.mul16_bits(x.view(np.uint16), y.view(np.uint16))).view(np.float16) == _f16_exact(fx * fy) or np.isinf(_f16_exact(fx * fy))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        (rng.standard_normal(20000) * 3000).astype(np.float32),
        rng.standard_normal(20000).astype(np.float32) * np.float32(1e-5),  # subnormal range
        np.float32([65504, 65519.99, 65520, 70000, -65520, 2.0 ** -25, 2.0 ** -24 * 1.5]),
        # exact ties between fp16 neighbours
        (np.arange(1, 2000, dtype=np.float32) * np.float32(2.0 ** -11) + np.float32(1.0)),
    ])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16_bits(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------------ fp32-state WKV


def _zeros16(B, T, C):
    return np.zeros((B, T, C), dtype=np.float16)


ORDERS = ["seq", "rows"]


@pytest.mark.parametrize("order", ORDERS)
def test_fp32_case_decay_only(order):
    """a=b=0, k=v=0: S' = S diag(d), y = S' r."""
    B, T, H = 1, 1, 2
    C = H * 64
    r, w, *_ = make_wkv_inputs(B, T, H, seed=3)
    S0 = make_state(B, H, seed=3, std=1.0)
    S = S0.copy()
    z = _zeros16(B, T, C)
    y = orc.wkv_fp32(B, T, C, H, S, r, w, z, z, z, z, order=order)
    d = decay64(w.astype(np.float64)).reshape(B, H, 64)
    S64 = S0.astype(np.float64) * d[:, :, None, :]
    np.testing.assert_allclose(S, S64, rtol=3e-7, atol=0)
    y64 = np.einsum("bhij,bhj->bhi", S64, r.astype(np.float64).reshape(B, H, 64)).reshape(B, T, C)
    np.testing.assert_allclose(y.astype(np.float64), y64, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("order", ORDERS)
def test_fp32_case_rank1_update(order):
    """a=b=0: S' = S diag(d) + v k^T (outer product)."""
    B, T, H = 1, 1, 1
    C = 64
    r, w, k, v, _, _ = make_wkv_inputs(B, T, H, seed=4)
    S0 = make_state(B, H, seed=4, std=1.0)
    S = S0.copy()
    z = _zeros16(B, T, C)
    orc.wkv_fp32(B, T, C, H, S, r, w, k, v, z, z, order=order)
    d = decay64(w.astype(np.float64))[0, 0]
    S64 = S0[0, 0].astype(np.float64) * d[None, :] + np.outer(v[0, 0].astype(np.float64), k[0, 0].astype(np.float64))
    np.testing.assert_allclose(S[0, 0], S64, rtol=1e-6, atol=1e-6)


def _delta_rule_case(seed):
    B, T, H = 1, 1, 1
    r, _, k, v, _, _ = make_wkv_inputs(B, T, H, seed=seed)
    g = np.random.default_rng(seed)
    kk = g.standard_normal(64)
    kk /= np.linalg.norm(kk)
    kk16 = kk.astype(np.float16).reshape(1, 1, 64)
    w = np.full((1, 1, 64), -np.inf, dtype=np.float16)  # decay exactly 1
    S0 = make_state(B, H, seed=seed, std=1.0)
    return r, w, k, v, kk16, S0


def _delta_rule_expect(S0, kk16, k, v):
    kk = kk16[0, 0].astype(np.float64)
    return S0[0, 0].astype(np.float64) @ (np.eye(64) - np.outer(kk, kk)) + np.outer(
        v[0, 0].astype(np.float64), k[0, 0].astype(np.float64))


@pytest.mark.parametrize("order", ORDERS)
def test_fp32_case_classic_delta_rule(order):
    """d=1, a=-kk, b=kk (unit kk): S' = S (I - kk kk^T) + v k^T."""
    r, w, k, v, kk16, S0 = _delta_rule_case(5)
    S = S0.copy()
    orc.wkv_fp32(1, 1, 64, 1, S, r, w, k, v, -kk16, kk16, order=order)
    np.testing.assert_allclose(S[0, 0], _delta_rule_expect(S0, kk16, k, v), rtol=1e-5, atol=2e-5)


def test_planted_mistake_is_caught_by_delta_rule_case():
    """A float64 restatement that drops the sa*b term must fail the delta-rule closed form."""
    r, w, k, v, kk16, S0 = _delta_rule_case(6)
    S = S0[0, 0].astype(np.float64)
    d = decay64(w.astype(np.float64))[0, 0]
    wrong = S * d[None, :] + np.outer(v[0, 0].astype(np.float64), k[0, 0].astype(np.float64))
    assert not np.allclose(wrong, _delta_rule_expect(S0, kk16, k, v), rtol=1e-5, atol=2e-5)


@pytest.mark.parametrize("order", ORDERS)
def test_fp32_case_zero_state_single_token(order):
    """S=0, T=1: y_i = v_i (k . r) per head."""
    B, T, H = 2, 1, 3
    C = H * 64
    r, w, k, v, a, b = make_wkv_inputs(B, T, H, seed=7)
    S = np.zeros((B, H, 64, 64), dtype=np.float32)
    y = orc.wkv_fp32(B, T, C, H, S, r, w, k, v, a, b, order=order)
    kr = (k.astype(np.float64) * r.astype(np.float64)).reshape(B, H, 64).sum(-1)
    want = v.astype(np.float64).reshape(B, H, 64) * kr[:, :, None]
    np.testing.assert_allclose(y.astype(np.float64).reshape(B, H, 64), want, rtol=2e-3, atol=2e-3)


def _wkv_fp32_float64(S, r, w, k, v, a, b):
    B, T, C = r.shape
    H = C // 64
    S = S.astype(np.float64).copy()
    y = np.zeros((B, T, C))
    for bi in range(B):
        for h in range(H):
            sl = slice(h * 64, h * 64 + 64)
            for t in range(T):
                rr, kk, vv, aa, bb = (x[bi, t, sl].astype(np.float64) for x in (r, k, v, a, b))
                d = decay64(w[bi, t, sl].astype(np.float64))
                St = S[bi, h]
                sa = St @ aa
                St = St * d[None, :] + np.outer(sa, bb) + np.outer(vv, kk)
                S[bi, h] = St
                y[bi, t, sl] = St @ rr
    return S, y


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("B,T,H,dist", [(1, 4, 1, "baseline"), (2, 3, 2, "realistic"), (1, 16, 1, "realistic")])
def test_fp32_matches_float64_brute_force(B, T, H, dist, order):
    C = H * 64
    ins = make_wkv_inputs(B, T, H, seed=11, dist=dist)
    S0 = make_state(B, H, seed=11)
    S = S0.copy()
    y = orc.wkv_fp32(B, T, C, H, S, *ins, order=order)
    S64, y64 = _wkv_fp32_float64(S0, *ins)
    np.testing.assert_allclose(S, S64, rtol=1e-4, atol=1e-4)
    # y is rounded to fp16: allow one fp16 ulp plus fp32 drift
    np.testing.assert_allclose(y.astype(np.float64), y64, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("order", ORDERS)
def test_fp32_prefill_equals_repeated_decode(order):
    B, T, H = 2, 9, 2
    C = H * 64
    ins = make_wkv_inputs(B, T, H, seed=12)
    S_seq = make_state(B, H, seed=12)
    S_one = S_seq.copy()
    y_seq = orc.wkv_fp32(B, T, C, H, S_seq, *ins, order=order)
    ys = [orc.wkv_fp32(B, 1, C, H, S_one, *(x[:, t:t + 1] for x in ins), order=order) for t in range(T)]
    assert np.array_equal(S_seq, S_one)
    assert np.array_equal(y_seq, np.concatenate(ys, axis=1))


def _sa_probe(cols):
    """One token with d = 1, k = v = r = 0, a = 1 on every column, b = e_63 and state row 0 =
    2^24 at column cols[0], 1 at cols[1] and cols[2] (column 63 zero): the updated S[0, 63]
    is exactly sa = the row's sum in the oracle's order."""
    S = np.zeros((1, 1, 64, 64), dtype=np.float32)
    S[0, 0, 0, cols[0]] = 2.0 ** 24
    S[0, 0, 0, cols[1]] = 1.0
    S[0, 0, 0, cols[2]] = 1.0
    ones = np.ones((1, 1, 64), dtype=np.float16)
    z = np.zeros((1, 1, 64), dtype=np.float16)
    w = np.full((1, 1, 64), -np.inf, dtype=np.float16)  # decay exactly 1
    b = z.copy()
    b[0, 0, 63] = 1.0
    return S, (z, w, z, z, ones, b)


# 2^24 + 1 is a tie that rounds (to even) back to 2^24; 2^24 + 2 is exact.  So the sum is
# 2^24 + 2 exactly when the two ones are added to each other before either meets 2^24.
# Row-split order: group g = columns 4g..4g+3, 32+4g..32+4g+3; tree ((0,1),(2,3)),((4,5),(6,7)).
DOT_PROBES = [
    ((0, 4, 36), 2.0 ** 24 + 2),  # 4 and 36 are both group 1: its chain adds the ones first
    ((0, 24, 28), 2.0 ** 24 + 2),  # groups 6 and 7 pair in the tree before the root
    ((0, 12, 16), 2.0 ** 24),      # groups 3 and 4 meet only at the root, after group 0 absorbed one
    ((0, 1, 33), 2.0 ** 24),       # all in group 0, 2^24 first in its chain
    ((0, 8, 12), 2.0 ** 24 + 2),   # groups 2 and 3 pair before meeting groups 0-1
]


@pytest.mark.parametrize("order", ORDERS)
@pytest.mark.parametrize("cols,rows_sum", DOT_PROBES)
def test_fp32_dot_order_known_answer(order, cols, rows_sum):
    """One chain from column 0 loses both ones (2^24); the row-split order gives rows_sum."""
    S, ins = _sa_probe(cols)
    orc.wkv_fp32(1, 1, 64, 1, S, *ins, order=order)
    want = 2.0 ** 24 if order == "seq" else rows_sum
    assert S[0, 0, 0, 63] == np.float32(want), (order, cols, S[0, 0, 0, 63])


def test_fp32_dot_order_planted_grouping_is_caught():
    """Eight contiguous columns per group (a plausible mistake) fails the first probe: 4 joins
    2^24's group, 36 sits in group 4, so both ones are absorbed."""
    cols, rows_sum = DOT_PROBES[0]
    row = np.zeros(64, dtype=np.float32)
    row[cols[0]], row[cols[1]], row[cols[2]] = 2.0 ** 24, 1.0, 1.0
    p = [np.float32(0)] * 8
    for j in range(64):
        p[j // 8] = np.float32(p[j // 8] + row[j])
    wrong = np.float32(np.float32(np.float32(p[0] + p[1]) + np.float32(p[2] + p[3]))
                       + np.float32(np.float32(p[4] + p[5]) + np.float32(p[6] + p[7])))
    assert wrong != np.float32(rows_sum)


def test_fp32_orders_agree_within_tolerance_and_differ_in_bits():
    B, T, H = 2, 32, 2
    C = H * 64
    ins = make_wkv_inputs(B, T, H, seed=14, dist="baseline")
    S1 = make_state(B, H, seed=14, std=0.1)
    S2 = S1.copy()
    y1 = orc.wkv_fp32(B, T, C, H, S1, *ins, order="seq")
    y2 = orc.wkv_fp32(B, T, C, H, S2, *ins, order="rows")
    assert np.abs(S1.astype(np.float64) - S2).max() <= 1e-5
    # y is rounded to fp16 from fp32 sums that differ by rounding only: at most one fp16 ulp
    y1d, y2d = y1.astype(np.float64), y2.astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(y1d), 2.0 ** -14))) - 10)
    assert (np.abs(y1d - y2d) <= ulp).all()
    assert not np.array_equal(S1, S2)


def test_fp32_orders_at_config0_meet_north_star_bounds():
    """BASELINE config 0 exactly (B=2, T=128, H=12, zero state, seed 0): the row-split order
    (the order of wkv_forward_fp32, mode 0, at 1 < T < 16, and of the mixed step's decode
    kernel) against the row-per-lane order of the reference's mode-0 kernel at this size
    (wkv_fp32_v2.cu:79-124, chosen by use_small_auto :212-226), both in the oracle: y within
    max-abs 2e-2 / mean-rel 5e-3, final state within 1e-3.  Measured: max-abs 0.015625 (one
    ulp at |y| in [16, 32)), mean-rel 1.6e-7, 223 of 196608 outputs differ, state max-abs
    9.5e-7.  (Where y is small through cancellation the two fp32 sums can be several fp16
    ulps of y apart; the bound is absolute.)  At config 0's T = 128 the GPU's mode 0 takes
    the chunked kernel, not the row-split one: that kernel's y is within 2e-2 where |y| < 32
    and within one fp16 ulp above (0.03125 at config 0: 281 of 196608 values off, mean-rel
    1.9e-7), checked on the GPU in tests/test_wkv_gpu.py."""
    B, T, H = 2, 128, 12
    C = H * 64
    ins = make_wkv_inputs(B, T, H, seed=0, dist="baseline")
    S_seq = make_state(B, H, seed=0, std=0.0)
    S_rows = S_seq.copy()
    y_seq = orc.wkv_fp32(B, T, C, H, S_seq, *ins, order="seq")
    y_rows = orc.wkv_fp32(B, T, C, H, S_rows, *ins, order="rows")
    a, b = y_seq.astype(np.float64), y_rows.astype(np.float64)
    err = np.abs(a - b)
    mean_rel = err.sum() / np.abs(a).sum()
    mismatches = int((y_seq.view(np.uint16) != y_rows.view(np.uint16)).sum())
    print(f"config 0 rows vs seq order: max-abs {err.max():.6g} mean-rel {mean_rel:.3g} "
          f">=1-ulp mismatches {mismatches}/{y_seq.size} state max-abs {np.abs(S_seq - S_rows).max():.3g}")
    assert err.max() <= 2e-2 and mean_rel <= 5e-3
    assert 0 < mismatches <= y_seq.size // 500
    assert np.abs(S_seq.astype(np.float64) - S_rows).max() <= 1e-3


def test_fp32_slots_leave_other_slots_untouched():
    P, B, H = 16, 5, 2
    C = H * 64
    pool = make_state(P, H, seed=13)
    before = pool.copy()
    slots = np.array([7, 2, 11, 0, 15], dtype=np.int64)
    ins = make_wkv_inputs(B, 1, H, seed=13)
    orc.wkv_fp32_slots(B, 1, C, H, pool, slots, *ins)
    other = np.setdiff1d(np.arange(P), slots)
    assert np.array_equal(pool[other], before[other])
    assert not np.array_equal(pool[slots], before[slots])


# ------------------------------------------------------------------ fp16-state WKV


def test_fp16_case_decay_only():
    """a=b=0, k=v=0 (fp16 family): S' = fp16(S*wd + S), y = fp16(y_even + y_odd)."""
    B, T, H = 1, 1, 1
    r, w, *_ = make_wkv_inputs(B, T, H, seed=21, dist="realistic")
    S0 = make_state(B, H, seed=21, std=0.5, dtype=np.float16)
    S = S0.copy()
    z = _zeros16(B, T, 64)
    el = np.array([5], dtype=np.int32)
    orc.wkv_fp16(B, T, 64, H, S, r, w, z, z, z, z, el)
    wd = np.array([orc.w_delta(float(w[0, 0, j]), 5 + j) for j in range(64)], dtype=np.uint16).view(np.float16)
    want = (S0[0, 0].astype(np.float64) * wd.astype(np.float64)[None, :] + S0[0, 0].astype(np.float64)).astype(np.float16)
    assert np.array_equal(S[0, 0], want)


def _wkv_fp16_float64(S, r, w, k, v, a, b, el, w0=None, legacy=False):
    B, T, C = r.shape
    H = C // 64
    S = S.astype(np.float64).reshape(B, H, 64, 64).copy()
    y = np.zeros((B, T, C))
    for bi in range(B):
        for h in range(H):
            sl = slice(h * 64, h * 64 + 64)
            for t in range(T):
                rr, kk, vv, aa, bb = (x[bi, t, sl].astype(np.float64) for x in (r, k, v, a, b))
                wf = w[bi, t, sl].astype(np.float64)
                if w0 is not None and not legacy:
                    wf = wf + w0.reshape(-1)[sl].astype(np.float64)
                wd = decay64(wf) - 1.0
                St = S[bi, h]
                sa = St @ aa
                St = St * (1.0 + wd)[None, :] + np.outer(sa, bb) + np.outer(vv, kk)
                S[bi, h] = St
                y[bi, t, sl] = St @ rr
    return S, y


@pytest.mark.parametrize("legacy", [False, True])
@pytest.mark.parametrize("with_w0", [False, True])
def test_fp16_matches_float64_brute_force(legacy, with_w0):
    if legacy and with_w0:
        pytest.skip("legacy op has no w0")
    B, T, H = 2, 6, 2
    C = H * 64
    ins = make_wkv_inputs(B, T, H, seed=22, dist="realistic")
    S0 = make_state(B, H, seed=22, std=0.1, dtype=np.float16)
    S = S0.copy()
    el = np.array([3, 100], dtype=np.int32)
    w0 = (np.random.default_rng(22).standard_normal(C) * 0.1).astype(np.float16) if with_w0 else None
    y = orc.wkv_fp16(B, T, C, H, S, *ins, el, w0=w0, legacy=legacy)
    S64, y64 = _wkv_fp16_float64(S0, *ins, el, w0=w0, legacy=legacy)
    # fp16 state: errors of a few fp16 ulps of values ~0.1-1; the dither is ~1e-3 of wd
    np.testing.assert_allclose(S.astype(np.float64).reshape(S64.shape), S64, rtol=2e-2, atol=2e-3)
    np.testing.assert_allclose(y.astype(np.float64), y64, rtol=2e-2, atol=1e-2)


@pytest.mark.parametrize("legacy", [False, True])
def test_fp16_prefill_equals_decode_with_advancing_phase(legacy):
    """seq(T) with elapsed e == T one-token calls with elapsed e+t (the dither phase adds t)."""
    B, T, H = 2, 5, 1
    C = 64
    ins = make_wkv_inputs(B, T, H, seed=23, dist="realistic")
    S_seq = make_state(B, H, seed=23, std=0.1, dtype=np.float16)
    S_one = S_seq.copy()
    el = np.array([7, 1 << 20], dtype=np.int32)
    y_seq = orc.wkv_fp16(B, T, C, H, S_seq, *ins, el, legacy=legacy)
    ys = []
    e = el.copy()
    for t in range(T):
        ys.append(orc.wkv_fp16(B, 1, C, H, S_one, *(x[:, t:t + 1] for x in ins), e, legacy=legacy))
        orc.advance_i32(e, 1)
    assert np.array_equal(S_seq, S_one)
    assert np.array_equal(y_seq, np.concatenate(ys, axis=1))


def test_fp16_phase_matters():
    """The dither makes elapsed_t observable (v1: per channel and token)."""
    B, T, H = 1, 3, 1
    ins = make_wkv_inputs(B, T, H, seed=24, dist="realistic")
    outs = []
    for e in (0, 12345):
        S = make_state(B, H, seed=24, std=0.1, dtype=np.float16)
        outs.append(orc.wkv_fp16(B, T, 64, H, S, *ins, np.array([e], dtype=np.int32)))
    assert not np.array_equal(outs[0], outs[1])


# ------------------------------------------------------------------ advance_i32


def test_advance_i32_exact():
    # reference tests/ops/test_v1_wkv_ops.py:409-436, plus wrap-around
    x = np.zeros(4, dtype=np.int32)
    orc.advance_i32(x, 5)
    assert (x == 5).all()
    orc.advance_i32(x, -10)
    assert (x == -5).all()
    y = np.array([2 ** 31 - 1, 0, -(2 ** 31)], dtype=np.int32)
    orc.advance_i32(y, 1)
    assert y.tolist() == [-(2 ** 31), 1, -(2 ** 31) + 1]
