"""Pins the oracle's SwiGLU step (oracle/ah_oracle_ffn.c) without running the reference:

* fixed_exp: the reference's own KATs and bounds (numeric/fixed_exp.rs zero_and_boundaries), its
  accuracy contract against exp on a grid (ACHIEVED_REL 1e-8 + 4 ulp on [-16, 21], the same
  bound the reference's accuracy test asserts), monotonicity, and the Horner loop's per-step
  rounding: to nearest by its error against the exact rational polynomial, ties away from zero
  on inputs where a step lands on a half (a floor, truncating or ties-to-even step fails them);
* silu_fixed: the reference's KATs (engine/tests.rs:949-963), the closed form v / (1 + e^-v) to
  within the exp tolerance, the saturation bounds and odd-symmetry-breaking sign handling;
* swiglu: the exact product rounding round_shift_32(silu * up) checked with Python big ints
  against silu values, and its overflow refusal;
* swiglu_quant_f32: the composition against quant_act of the element-wise results.
"""
import math

import numpy as np

import oracle

ONE = 1 << 32
LN2_Q32 = 2977044472
I64_MAX, I64_MIN = (1 << 63) - 1, -(1 << 63)


def test_fixed_exp_reference_kats_and_bounds():
    assert oracle.fixed_exp(0) == (0, ONE)
    assert oracle.fixed_exp(-16 * ONE)[0] == 0 and oracle.fixed_exp(21 * ONE)[0] == 0
    assert oracle.fixed_exp(-16 * ONE - 1)[0] == 13
    assert oracle.fixed_exp(21 * ONE + 1)[0] == 13
    assert oracle.fixed_exp(I64_MIN)[0] == 13 and oracle.fixed_exp(I64_MAX)[0] == 13


def test_fixed_exp_accuracy_and_monotone():
    step = ONE // 1024 * 37  # a coarser grid than the reference's ONE/1024, same window
    prev = None
    for x in range(-16 * ONE, 21 * ONE + 1, step):
        st, v = oracle.fixed_exp(x)
        assert st == 0
        want = math.exp(x / ONE)
        got = v / ONE
        assert abs(got - want) <= 1e-8 * want + 4.0 / ONE, (x, got, want)
        if prev is not None:
            assert v >= prev
        prev = v


def test_silu_reference_kats():
    # engine/tests.rs:949-963
    assert oracle.silu_fixed(0) == (0, 0)
    assert oracle.silu_fixed(LN2_Q32) == (0, 1_984_696_315)
    assert oracle.silu_fixed(-LN2_Q32) == (0, -992_348_157)
    assert oracle.silu_fixed(16 * ONE) == (0, 16 * ONE)
    assert oracle.silu_fixed(16 * ONE + 1) == (0, 16 * ONE + 1)
    assert oracle.silu_fixed(-21 * ONE) == (0, 0)
    assert oracle.silu_fixed(-21 * ONE - 1) == (0, 0)
    assert oracle.silu_fixed(I64_MIN) == (0, 0)
    assert oracle.silu_fixed(I64_MAX) == (0, I64_MAX)


def test_silu_closed_form():
    rng = np.random.default_rng(3)
    xs = list(rng.integers(-21 * ONE + 1, 16 * ONE, size=3000)) + [1, -1, 2 ** 20, -(2 ** 20)]
    for v in xs:
        v = int(v)
        st, s = oracle.silu_fixed(v)
        assert st == 0
        r = v / ONE
        want = r / (1.0 + math.exp(-r))
        # exp carries ~1e-8 relative error (+4 ulp); silu inherits it through the quotient
        assert abs(s / ONE - want) <= 2e-8 * abs(want) + 4.0 / ONE * (1 + abs(r)), (v, s / ONE, want)
        assert (s >= 0) == (v >= 0) or s == 0


def test_swiglu_exact_rounding_and_overflow():
    rng = np.random.default_rng(4)
    for _ in range(3000):
        g = int(rng.integers(-30 * ONE, 30 * ONE))
        u = int(rng.integers(-(1 << 62), 1 << 62)) >> int(rng.integers(0, 40))
        st, s = oracle.silu_fixed(g)
        assert st == 0
        want = (s * u + (1 << 31)) >> 32  # Python big ints: floor of (prod + 2^31) / 2^32
        st2, h = oracle.swiglu(g, u)
        if I64_MIN <= want <= I64_MAX:
            assert st2 == 0 and h == want, (g, u)
        else:
            assert st2 == 12
    assert oracle.swiglu(20 * ONE, 1 << 62)[0] == 12  # 20 * 2^62 leaves i64


def test_swiglu_quant_f32_composition():
    rng = np.random.default_rng(5)
    n = 300
    gate = (rng.standard_normal(n) * 4).astype(np.float32)
    up = rng.standard_normal(n).astype(np.float32)
    gate[:7] = [0.0, -30.0, 20.0, 16.0, -21.0, 1e-9, -1e-9]
    st, codes, scales, h = oracle.swiglu_quant_f32(gate, up)
    assert st == 0
    for i in range(n):
        g = oracle.to_q32(int(gate[i:i + 1].view(np.uint32)[0]))[1]
        u = oracle.to_q32(int(up[i:i + 1].view(np.uint32)[0]))[1]
        assert h[i] == oracle.swiglu(g, u)[1]
    st2, c2, s2 = oracle.quant_act(h)
    assert st2 == 0 and (c2 == codes).all() and (s2 == scales).all()
    bad = gate.copy()
    bad[10] = np.inf
    assert oracle.swiglu_quant_f32(bad, up)[0] == 10


def _horner_exact(r):
    """exp's degree-7 Taylor polynomial at r / 2^32 in Q32.32, evaluated without rounding: the
    coefficients are round(2^32 / j!) (the reference's table, numeric/fixed_exp.rs:68-84), each
    Horner step acc * r / 2^32 + c exact in rationals."""
    from fractions import Fraction
    c = [round(Fraction(ONE, math.factorial(7 - i))) for i in range(8)]
    h = Fraction(c[0])
    for i in range(1, 8):
        h = h * r / ONE + c[i]
    return h, c


def _horner_rounded(r, tie_away):
    """The same evaluation with each step rounded to the nearest integer, ties away from zero or
    to even: the two readings of 'round' whose difference the oracle must resolve."""
    from fractions import Fraction
    _, c = _horner_exact(0)
    acc = c[0]
    for i in range(1, 8):
        p = Fraction(acc * r, ONE)
        fl = p.numerator // p.denominator
        frac = p - fl
        if frac > Fraction(1, 2) or (frac == Fraction(1, 2) and (p > 0 if tie_away else fl % 2 == 1)):
            fl += 1
        acc = fl + c[i]
    return acc


def test_fixed_exp_horner_rounds_each_step_to_nearest():
    """The per-step rounding of fixed_exp's Horner loop, pinned by its error against the exact
    polynomial.  At k = 0 (|x| < ln2 / 2) the output is the Horner result itself.  Rounding each
    of the 7 steps to nearest leaves |out - exact| <= 1/2 * sum_j |r|^j (|r| < 0.35 in units of
    one, each earlier error shrunk by the later multiplications) with an error mean near 0; a
    floor or truncating step errs by up to a whole unit per step, one-sided, and fails both."""
    rng = np.random.default_rng(11)
    half_ln2 = LN2_Q32 // 2
    xs = [int(v) for v in rng.integers(-half_ln2 + 1, half_ln2, size=4000)]
    xs += [1, -1, 2, -2, half_ln2 - 1, -half_ln2 + 1, 1 << 27, -(1 << 27)]
    errs = []
    for x in xs:
        st, v = oracle.fixed_exp(x)
        assert st == 0
        exact, _ = _horner_exact(x)
        t = abs(x) / ONE
        bound = 0.5 * sum(t ** j for j in range(7)) + 1e-9
        err = float(v - exact)
        assert abs(err) <= bound, (x, err, bound)
        errs.append(err)
    assert abs(sum(errs) / len(errs)) < 0.05, sum(errs) / len(errs)


def test_fixed_exp_horner_ties_away_from_zero():
    """Inputs where some Horner step lands exactly on a half and the two tie rules then give
    different outputs: the oracle takes ties away from zero, as the reference's round_div_2p32
    does (numeric/fixed_exp.rs:68-84).  The inputs were found by searching multiples of 2^18
    (positive) and 2^14 (negative; such ties that survive to the output are rare there) for a
    difference between the two rules; the test re-derives that they differ."""
    for x in (799539200, 805306368, 1375731712, -751026176):
        away, even = _horner_rounded(x, True), _horner_rounded(x, False)
        assert away != even, x
        st, v = oracle.fixed_exp(x)
        assert st == 0 and v == away, (x, v, away, even)
