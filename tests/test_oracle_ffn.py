"""Pins the oracle's SwiGLU step (oracle/ah_oracle_ffn.c) without running the reference:

* fixed_exp: the reference's own KATs and bounds (numeric/fixed_exp.rs zero_and_boundaries), its
  accuracy contract against exp on a grid (ACHIEVED_REL 1e-8 + 4 ulp on [-16, 21], the same
  bound the reference's accuracy test asserts) and monotonicity;
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
