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
