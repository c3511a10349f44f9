"""Integer identities the HIP kernels rely on, checked against the oracle on the CPU.

* the activation-scale exponent by bit length (ah_act_scale_exp) equals act_scale
  (kern/pow2.rs:11-39) -- the kernels avoid a 64-bit division by 127;
* the GEMM's exact f16 operands: every int8 code, Q4_K sc*q (<= 945) and Q6_K u-32 is an
  integer f16 represents exactly, and the split X = 64*floor(X/64) + (X mod 64) of a 32-code sum
  is exact in two f16 pieces.
"""
import numpy as np

import oracle


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


def act_code_f32_float(bits: int, e: int) -> int:
    """The kernels' f32-arithmetic code (quad_quant's fast path, e <= 55), on numpy float32:
    v = |x| * 2^(32-e) exact, code = trunc(fl(v + 0.5)); below 2^-9 to_q32's rounding first."""
    a = bits & 0x7FFFFFFF
    f = np.array([a], np.uint32).view(np.float32)[0]
    if a != 0 and a < (118 << 23):
        q = np.floor(np.float32(f * np.float32(2.0 ** 32)) + np.float32(0.5))
        v = np.float32(q * np.float32(np.ldexp(1.0, -e)))
    else:
        v = np.float32(f * np.float32(np.ldexp(1.0, 32 - e)))
    c = int(np.float32(v + np.float32(0.5)))
    return -c if bits >> 31 else c


def test_act_code_f32_float_path_matches_quant_act():
    """The same sweep for the float form: every element of every block whose exponent admits it
    (e <= 55) gets quant_act_f32's code."""
    rng = np.random.default_rng(18)
    blocks = []
    for top in list(range(-60, 24)) + [-126, -149]:
        amax = np.float32(np.ldexp(1.0 + rng.random(), top)) if top > -149 else np.float32(np.ldexp(1.0, -149))
        for _ in range(6):
            rel = rng.integers(-40, 1, size=31)
            body = np.ldexp(rng.random(31) + 0.5, top + rel).astype(np.float32)
            body *= np.where(rng.random(31) < 0.5, -1, 1).astype(np.float32)
            body[0] = np.float32(np.ldexp(1.5, top - 6))
            body[1] = np.float32(np.ldexp(0.5, -32))
            body[2] = np.float32(-np.ldexp(1.5, -33))
            body[3] = np.float32(0.0)
            body[4] = np.float32(-0.0)
            body[5] = np.float32(np.ldexp(1.0, -149))
            # half-way points of the code rounding just below 2^-9 (two roundings) and above it
            body[6] = np.float32(np.ldexp(1.0, -9) * (1 - 2 ** -24))
            body[7] = np.float32(np.ldexp(1.0, -9))
            blocks.append(np.concatenate([[amax], body]).astype(np.float32))
    # N(0,1) activations, the common case
    blocks.append(rng.standard_normal(32 * 400).astype(np.float32))
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
        if e > 55:
            continue
        assert act_code_f32_float(int(bits[i]), e) == int(codes[i]), (i, float(x[i]), e)
        n_checked += 1
    assert n_checked > 25000
