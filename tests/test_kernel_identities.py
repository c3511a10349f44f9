"""Integer identities the HIP kernels rely on, checked against the oracle on the CPU.

* the activation-scale exponent by bit length (ah_act_scale_exp) equals act_scale
  (kern/pow2.rs:11-39) -- the kernels avoid a 64-bit division by 127;
* the GEMM's exact f16 operands: every int8 code, Q4_K sc*q (<= 945) and Q6_K u-32 is an
  integer f16 represents exactly, and the split X = 64*floor(X/64) + (X mod 64) of a 32-code sum
  is exact in two f16 pieces;
* the f32 quantizer's two forms, the 32-bit integer one (ah_act_code_f32) and the f32-arithmetic
  one (quad_quant_f32: exponent from the largest magnitude's bits, codes by one fma rounding,
  cleared below half a code unit, a second rounding below 2^-9 at exponents <= 24), against
  quant_act_f32, with a brute force over every f32 of the fma's sum.
"""
import numpy as np

import oracle
from quant_edges import edge_blocks_f32


def act_scale_exp_by_bitlength(a: int) -> int:
    if a == 0:
        return -1
    b = a.bit_length()
    e0 = b - 7 if b > 7 else 0
    e = e0 + (1 if a > (127 << e0) else 0)
    return 63 if e > 62 else e


def test_act_scale_exponent_identity():
    rng = np.random.default_rng(9)
    vals = [1, 126, 127, 128, 129, 254, 255, 256, (1 << 64) - 1, 1 << 63, (1 << 63) - 1,
            127 << 56, (127 << 56) + 1]
    for k in range(1, 64):
        for d in (-2, -1, 0, 1, 2):
            vals.append(max(1, (1 << k) + d))
            vals.append(max(1, (127 << max(0, k - 7)) + d))
    vals += [int(v) | 1 for v in rng.integers(1, 1 << 63, size=5000, dtype=np.uint64)]
    vals += [int(v) >> int(s) for v, s in zip(rng.integers(1, 1 << 63, size=5000, dtype=np.uint64),
                                              rng.integers(0, 62, size=5000))]
    for a in vals:
        if a == 0:
            continue
        s = oracle.act_scale(a)
        want = 63 if s is None else s.bit_length() - 1
        assert act_scale_exp_by_bitlength(a) == want, a


def test_gemm_operands_exact_in_f16():
    q8 = np.arange(-128, 128)
    assert (q8.astype(np.float16).astype(np.int64) == q8).all()
    sc_q = np.array([s * q for s in range(64) for q in range(16)])
    assert (sc_q.astype(np.float16).astype(np.int64) == sc_q).all()
    u6 = np.arange(64) - 32
    assert (u6.astype(np.float16).astype(np.int64) == u6).all()
    X = np.arange(-127 * 32, 127 * 32 + 1)
    hi = 64 * np.floor_divide(X, 64)
    lo = X - hi
    assert ((hi.astype(np.float16).astype(np.int64) + lo.astype(np.float16).astype(np.int64)) == X).all()
    assert lo.min() >= 0 and lo.max() <= 63


def act_code_f32_32bit(bits: int, e: int) -> int:
    """The kernels' 32-bit per-element code (ah_act_code_f32), restated on Python ints."""
    eb = (bits >> 23) & 0xFF
    ee = eb if eb else 1
    m = (bits & 0x7FFFFF) | (0x800000 if eb else 0)
    if ee >= 118:
        sh = e + 118 - ee
        k = 0 if sh < 1 else min(sh - 1, 25)
        c = ((m >> k) + 1) >> 1
    else:
        k1 = min(117 - ee, 25)
        mag = ((m >> k1) + 1) >> 1
        k = 0 if e < 1 else min(e - 1, 25)
        c = mag if e == 0 else ((mag >> k) + 1) >> 1
    return -c if bits >> 31 else c


def test_act_code_f32_32bit_matches_quant_act():
    """Blocks of 32 f32 values: element 0 sets the block's scale, the rest sweep every exponent the
    scale admits (tiny values that round twice, half-way points, subnormals, signed zeros); the
    32-bit code must equal quant_act_f32's (kern/quant.rs via the oracle) for every element."""
    rng = np.random.default_rng(17)
    blocks = []
    for top in list(range(-60, 31)) + [-126, -149]:
        amax = np.float32(np.ldexp(1.0 + rng.random(), top)) if top > -149 else np.float32(np.ldexp(1.0, -149))
        for _ in range(6):
            rel = rng.integers(-40, 1, size=31)
            body = np.ldexp(rng.random(31) + 0.5, top + rel).astype(np.float32)
            body *= np.where(rng.random(31) < 0.5, -1, 1).astype(np.float32)
            # exact half-way points of the code rounding and of to_q32's rounding
            body[0] = np.float32(np.ldexp(1.5, top - 6))
            body[1] = np.float32(np.ldexp(0.5, -32))
            body[2] = np.float32(-np.ldexp(1.5, -33))
            body[3] = np.float32(0.0)
            body[4] = np.float32(-0.0)
            body[5] = np.float32(np.ldexp(1.0, -149))
            blocks.append(np.concatenate([[amax], body]).astype(np.float32))
    x = np.concatenate(blocks)
    st, codes, scales = oracle.quant_act_f32(x)
    assert st == 0
    bits = x.view(np.uint32)
    n_checked = 0
    for i in range(x.shape[0]):
        s = int(scales[i // 32])
        if s == 0:
            continue
        e = s.bit_length() - 1
        assert act_code_f32_32bit(int(bits[i]), e) == int(codes[i]), (i, float(x[i]), e)
        n_checked += 1
    assert n_checked > 15000


def test_code_rounding_by_float_sum_brute_force():
    """Every f32 v in [2^-26, 128): trunc(fl(v + 1/2)) = floor(v + 1/2) (exact in f64) for
    v >= 1/2, and below 1/2 the one exception is v = 1/2 - 2^-25 (rounded up to 1, a tie to
    even), which quad_quant_f32 clears with its |x| >= 2^(e-33) compare."""
    bad = []
    for binade in range(-26, 7):
        m = np.arange(1 << 23, dtype=np.uint32)
        v = ((np.uint32(binade + 127) << np.uint32(23)) | m).view(np.float32)
        got = np.trunc(v + np.float32(0.5))
        want = np.floor(v.astype(np.float64) + 0.5)
        bad.extend(float(t) for t in v[got != want])
    assert bad == [0.5 - 2.0 ** -25]


def quad_quant_f32_block(bits: np.ndarray, second: bool = True, clear: bool = True):
    """quad_quant_f32 on one 32-block of f32 bit patterns, restated on numpy float32: None outside
    its common case (a largest magnitude outside [2^-9, 2^29) and nonzero), else (e, codes).
    The exponent comes from the largest magnitude's bits, e = ee - 101 + [m > 0xFE0000]; each code
    is trunc(fl(x * 2^(32-e) + copysign(1/2, x))) (x * 2^(32-e) is exact, so the numpy product and
    sum are the kernel's one fma rounding), 0 where |x| < 2^(e-33) (with `clear`); with `second`,
    elements below 2^-9 take to_q32's rounding first, q = floor(fl(|x| * 2^32 + 1/2)), then code = trunc(fl(q * 2^-e + 1/2))."""
    bits = np.asarray(bits, np.uint32)
    a = bits & np.uint32(0x7FFFFFFF)
    maxb = int(a.max())
    if not (maxb == 0 or 0x3B000000 <= maxb < 0x4E000000):
        return None
    e = -1 if maxb == 0 else (maxb >> 23) - 101 + (1 if (maxb & 0x7FFFFF) > 0x7E0000 else 0)
    x = bits.view(np.float32)
    half = ((bits & np.uint32(0x80000000)) | np.uint32(0x3F000000)).view(np.float32)
    codes = np.trunc(x * np.float32(np.ldexp(1.0, 32 - e)) + half).astype(np.int64)
    if clear:
        codes = np.where(np.abs(x) >= np.float32(np.ldexp(1.0, e - 33)), codes, 0)
    if second:
        fa = a.view(np.float32)
        q = np.floor(fa * np.float32(2.0 ** 32) + np.float32(0.5))
        cm = np.trunc(q * np.float32(np.ldexp(1.0, -e)) + np.float32(0.5)).astype(np.int64)
        tiny = a < np.uint32(0x3B000000)
        codes = np.where(tiny, np.where(bits >> 31 != 0, -cm, cm), codes)
    return e, codes


def test_act_code_f32_fast_block_matches_quant_act():
    """Every block of a sweep that quad_quant_f32 accepts gets quant_act_f32's exponent and codes;
    at e >= 25 the second rounding is not needed (the kernel runs it only in waves holding a block
    at e <= 24) and is harmless where it runs; at e = 24 it is needed."""
    x = edge_blocks_f32(np.random.default_rng(18))
    st, codes, scales = oracle.quant_act_f32(x)
    assert st == 0
    bits = x.view(np.uint32)
    n_blocks = n_second = n_clear = 0
    for bi in range(x.shape[0] // 32):
        got = quad_quant_f32_block(bits[32 * bi:32 * bi + 32])
        if got is None:
            continue
        s = int(scales[bi])
        want_e = -1 if s == 0 else s.bit_length() - 1
        want = codes[32 * bi:32 * bi + 32].astype(np.int64)
        assert got[0] == want_e, (bi, got[0], want_e)
        assert (got[1] == want).all(), (bi, want_e)
        if (quad_quant_f32_block(bits[32 * bi:32 * bi + 32], clear=False)[1] != want).any():
            n_clear += 1
        one = quad_quant_f32_block(bits[32 * bi:32 * bi + 32], second=False)[1]
        if want_e >= 25:
            assert (one == want).all(), (bi, want_e)
        elif (one != want).any():
            n_second += 1
        n_blocks += 1
    assert n_blocks > 500
    assert n_second > 0  # the second rounding decides some code at e <= 24
    assert n_clear >= 4  # and the clear below half a unit some code at each sampled e


# ---- the fused FFN's exp in i64 (fx_exp in ah_swiglu.h) -------------------------------------------

_EXP_C = [852176, 5965232, 35791394, 178956971, 715827883, 2147483648, 4294967296, 4294967296]
I64_MAX, I64_MIN = (1 << 63) - 1, -(1 << 63)


def _rdiv32(v: int) -> int:
    """round(v / 2^32), ties away from zero: the device's branch-free i64 form (valid for
    |v| <= 2^63 - 2^31)."""
    assert -(1 << 63) + (1 << 31) <= v <= (1 << 63) - (1 << 31), v
    a = -v if v < 0 else v
    q = (a + (1 << 31)) >> 32
    return -q if v < 0 else q


def fx_exp_i64(x: int):
    """The device's exp(x) in Q32.32, step for step, asserting that every product of its Horner
    sum is an i64 (the reason the reference's i128 sum may run in i64 there)."""
    if x < -16 * (1 << 32) or x > 21 * (1 << 32):
        return 13, 0
    k = (x * 6196328019 + (1 << 63)) >> 64
    r = x - k * 2977044472
    assert abs(r) < 1 << 31
    acc = _EXP_C[0]
    for c in _EXP_C[1:]:
        p = acc * r
        assert I64_MIN <= p <= I64_MAX, (x, acc, r)
        acc = _rdiv32(p) + c
        assert 0 < acc < (1 << 33), (x, acc)
    if k >= 0:
        if k >= 63 or acc > (I64_MAX >> k) or acc < (I64_MIN >> k):
            return 13, 0
        return 0, acc << k
    n = -k
    return 0, (0 if n >= 63 else (acc + (1 << (n - 1))) >> n)


def test_fx_exp_i64_equals_fixed_exp():
    """fx_exp's i64 Horner equals the reference's i128 one (oracle aho_fixed_exp, pinned by the
    reference's KATs in test_oracle_ffn.py) across the whole domain: every half-way point of
    k = round(x / ln 2) (where |r| is largest) with its neighbours, the range ends, powers of two
    and a random sweep; no product leaves i64 on the way."""
    one = 1 << 32
    xs = [-16 * one, 21 * one, -16 * one - 1, 21 * one + 1, 0, 1, -1, one, -one]
    ln2 = 2977044472
    for k in range(-24, 32):
        mid = (2 * k + 1) * ln2 // 2
        xs += [mid + d for d in range(-3, 4)] + [k * ln2 + d for d in (-1, 0, 1)]
    for e in range(0, 37):
        xs += [1 << e, -(1 << e), (1 << e) - 1]
    rng = np.random.default_rng(0xE4B)
    xs += [int(v) for v in rng.integers(-16 * one, 21 * one, size=20000, dtype=np.int64)]
    for x in xs:
        assert fx_exp_i64(x) == tuple(oracle.fixed_exp(x)), x


def silu_one_step(v: int):
    """The device's silu (silu_fx in ah_swiglu.h) step for step: the f64 estimate of the rounded
    quotient, truncated, then ONE correction against the exact remainder; also returns how far the
    truncated estimate was from the exact quotient."""
    one = 1 << 32
    if v >= 16 * one:
        return v, 0
    if v <= -21 * one:
        return 0, 0
    st, e = fx_exp_i64(-v)
    assert st == 0
    den = one + e
    mag = -v if v < 0 else v
    n2 = mag * one + (den >> 1)
    nd = float(n2 >> 32) * 4294967296.0 + float(n2 & 0xFFFFFFFF)  # each term exact; one rounding
    q0 = int(nd / float(den))                                       # truncation toward zero
    rem = n2 - q0 * den
    q = q0 + (-1 if rem < 0 else 1 if rem >= den else 0)
    return (-q if v < 0 else q), q0 - n2 // den


def test_silu_single_correction_is_exact():
    """One correction step after the f64 estimate gives the exact rounded quotient (the oracle's
    i128 division, pinned by the reference's values in test_oracle_ffn.py): over the saturation
    bounds, the exp range reduction's half-way points, small and large magnitudes and a random
    sweep, the corrected quotient equals the oracle's and the estimate was never off by more
    than one."""
    one = 1 << 32
    vs = [16 * one - 1, 16 * one, -21 * one + 1, -21 * one, 0, 1, -1, one, -one, 15 * one, -20 * one]
    ln2 = 2977044472
    for k in range(-24, 32):
        mid = (2 * k + 1) * ln2 // 2
        vs += [-(mid + d) for d in range(-2, 3)]
    for e in range(0, 36):
        vs += [1 << e, -(1 << e)]
    rng = np.random.default_rng(0x5117)
    vs += [int(v) for v in rng.integers(-21 * one, 16 * one, size=50000, dtype=np.int64)]
    for v in vs:
        got, off = silu_one_step(v)
        st, ref = oracle.silu_fixed(v)
        assert st == 0 and got == ref and abs(off) <= 1, (v, off)
