"""Pins the C oracle before anything is checked against it.

Each oracle function is compared with (a) the reference's own known-answer tests, restated
here with their file:line, (b) this project's independent big-integer brute force
(tests/golden/bruteforce.py), and (c) invariants the mathematics fixes.
"""
import numpy as np
import pytest

import bruteforce as bf
import oracle
from apeiron_amd import synth

ONE = 1 << 32
I64_MIN, I64_MAX = -(1 << 63), (1 << 63) - 1


def test_f16_to_fixed_exhaustive():
    # chart/tests.rs:85-102 checks all 65536 words; here against an exact rational decode.
    for h in range(65536):
        st, v = oracle.f16_to_fixed(h)
        want = bf.f16_q32(h)
        if want is None:
            assert st == 6, hex(h)  # NonFiniteScale
        else:
            assert st == 0 and v == want, hex(h)


def _f32_words(rng, n):
    edge = [0, 0x80000000, 1, 0x80000001, 0x007FFFFF, 0x00800000, 0x3F800000, 0xBF800000,
            0x2F800000, 0x2F000000, 0x2EFFFFFF, 0x2F000001, 0xAF000000, 0x30000000,
            0x4EFFFFFF, 0x4F000000, 0xCF000000, 0xCF000001, 0x7F7FFFFF, 0x7F800000,
            0xFF800000, 0x7FC00000, 0x33800000, 0x34000000, 0x33FFFFFF]
    # ties: v*2^32 = k + 1/2 at small exponents
    for k in range(1, 40):
        edge.append(int(np.array([np.float32((2 * k + 1) / 2 ** 33)]).view(np.uint32)[0]))
        edge.append(int(np.array([np.float32(-(2 * k + 1) / 2 ** 33)]).view(np.uint32)[0]))
    rnd = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).tolist()
    normals = rng.standard_normal(n).astype(np.float32).view(np.uint32).tolist()
    return edge + rnd + normals


def test_to_q32_against_exact_rounding():
    rng = np.random.default_rng(7)
    for w in _f32_words(rng, 4000):
        st, v = oracle.to_q32(w)
        f = np.array([w], dtype=np.uint32).view(np.float32)[0]
        want = bf.f32_q32(w)
        if not np.isfinite(f):
            assert st == 10, hex(w)
        elif want is None:
            assert st == 11, hex(w)
        else:
            assert st == 0 and v == want, hex(w)


def test_act_scale_reference_samples_and_bruteforce():
    # kern/pow2.rs:105-135 sample table and its properties.
    samples = [0, 1, 126, 127, 128, 254, 255, 1 << 20, (1 << 20) + 1, 127 << 40, (127 << 40) + 1,
               127 << 56, (127 << 56) + 1, (1 << 64) - 1]
    rng = np.random.default_rng(3)
    samples += [int(v) for v in rng.integers(0, 1 << 63, size=300, dtype=np.uint64)]
    for a in samples:
        s = oracle.act_scale(a)
        c = -(-a // 127)
        if s is None:
            assert c > (1 << 62), a
            continue
        if s == 0:
            assert a == 0
            continue
        assert s & (s - 1) == 0
        assert s * 127 >= a
        assert s == 1 or (s // 2) * 127 < a
        assert s < 2 * max(c, 1)
        assert s == bf.least_pow2_scale(a)


def test_quant_act_reference_kats():
    # chart/tests.rs:397-415
    st, codes, scales = oracle.quant_act([3, 130, -3])
    assert st == 0 and codes[0] == 2 and codes[2] == -2 and scales[0] == 2
    st, codes, scales = oracle.quant_act([0] * 64)
    assert st == 0 and not codes.any() and not scales.any()
    st, _, _ = oracle.quant_act([I64_MAX] * 32)
    assert st == 7  # FixedOverflow: code 64 * 2^57 leaves i64
    st, codes, scales = oracle.quant_act([I64_MIN] * 32)
    assert st == 0 and scales.tolist() == [1 << 57]
    st, xhat = oracle.dequant_act(codes, scales)
    assert st == 0 and xhat.tolist() == [I64_MIN] * 32
    st, codes, scales = oracle.quant_act([127 << 56] * 32)
    assert st == 0
    assert oracle.dequant_act(codes, scales)[1].tolist() == [127 << 56] * 32


def test_quant_act_invariants_and_bruteforce():
    # chart/tests.rs:373-395 properties, plus equality with the brute force.
    for seed in range(16):
        rng = np.random.default_rng(0x5EED1000 + seed)
        x = ((rng.integers(0, 4096, size=200) - 2048) * 1_000_003).astype(np.int64)
        st, codes, scales = oracle.quant_act(x)
        assert st == 0
        assert codes.shape == (200,) and scales.shape == (7,)
        xhat = oracle.dequant_act(codes, scales)[1]
        for j, xv in enumerate(x.tolist()):
            s = int(scales[j // 32])
            assert abs(int(codes[j])) <= 127
            if s == 0:
                assert codes[j] == 0
            assert 2 * abs(xv - int(xhat[j])) <= s
        ref = bf.quant_act(x.tolist())
        assert codes.tolist() == ref[0] and scales.tolist() == ref[1]
    # wide magnitude spread, zero blocks, ragged tail
    rng = np.random.default_rng(11)
    x = [0] * 32 + [int(v) for v in rng.integers(-(1 << 62), 1 << 62, size=71)]
    st, codes, scales = oracle.quant_act(x)
    ref = bf.quant_act(x)
    assert st == 0 and codes.tolist() == ref[0] and scales.tolist() == ref[1]


def test_quant_act_f32_matches_bruteforce():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(896).astype(np.float32)
    x[:32] = 0
    x[40] = 1e-12
    st, codes, scales = oracle.quant_act_f32(x)
    q = [bf.f32_q32(int(w)) for w in x.view(np.uint32)]
    ref = bf.quant_act(q)
    assert st == 0 and codes.tolist() == ref[0] and scales.tolist() == ref[1]
    assert oracle.quant_act_f32(np.array([np.inf], np.float32))[0] == 10
    assert oracle.quant_act_f32(np.array([3e9], np.float32))[0] == 11


def test_format_unpack_kats():
    # format/quant.rs:873-883: Q4_K codes[0]=3, codes[32]=0xA, pair (5,7) -- read through the
    # dequantizer with d = dmin = 1.0 so w = sc*q - m.
    blk = np.zeros(144, np.uint8)
    blk[0:2] = [0x00, 0x3C]
    blk[2:4] = [0x00, 0x3C]
    blk[4], blk[8], blk[16] = 5, 7, 0xA3
    st, w = oracle.dequant_row(12, blk, 256)
    assert st == 0
    assert w[0] == (5 * 3 - 7) * ONE
    # sub-block 1 (high nibble) uses pair 1 = (scales[1]&63, scales[5]&63) = (0, 0)
    assert w[32] == 0
    # format/quant.rs:886-897: Q6_K codes[0] = -15, codes[32] = -32, with d = 1, sc = 1
    b6 = np.zeros(210, np.uint8)
    b6[0], b6[128] = 0x01, 0x01
    b6[192:208] = 1
    b6[208:210] = [0x00, 0x3C]
    st, w = oracle.dequant_row(14, b6, 256)
    assert st == 0 and w[0] == -15 * ONE and w[32] == -32 * ONE
    # Q8_0 (format/quant.rs:858-869): d = 0.5, codes 2 and -2
    b8 = np.zeros(34, np.uint8)
    b8[0:2] = [0x00, 0x38]
    b8[2], b8[3] = 2, 0xFE
    st, w = oracle.dequant_row(8, b8, 32)
    assert st == 0 and w[0] == ONE and w[1] == -ONE
    # Q5_0 (format/quant.rs:836-857): d = 0.5; qh[0] = 0b101 sets the fifth bit of outputs 0 and 2,
    # qh[2] = 1 that of output 16; qs[0] = 0xFF, qs[1] = 0, qs[2] = 0x10
    b5 = np.zeros(22, np.uint8)
    b5[0:2] = [0x00, 0x38]
    b5[2], b5[4] = 0b101, 1
    b5[6], b5[7], b5[8] = 0xFF, 0x00, 0x10
    st, w = oracle.dequant_row(6, b5, 32)
    assert st == 0
    got = {i: int(w[i]) // (ONE // 2) for i in (0, 1, 2, 3, 16, 17, 18)}
    assert got == {0: 15, 1: -16, 2: 0, 3: -16, 16: 15, 17: -16, 18: -15}
    assert bf.q5_0_codes(bytes(b5))[:4] == [15, -16, 0, -16]
    # engine/tests.rs:60-72: d = 1.0, qh[2] = 1, qs[0] = 0x21 -> w[0] = -15, w[1] = -16,
    # w[16] = (2 | 16) - 16 = 2, w[17] = -16
    b5 = np.zeros(22, np.uint8)
    b5[0:2] = [0x00, 0x3C]
    b5[4], b5[6] = 0x01, 0x21
    st, w = oracle.dequant_row(6, b5, 32)
    assert st == 0 and len(w) == 32
    assert (w[0], w[1], w[16], w[17]) == (-15 * ONE, -16 * ONE, 2 * ONE, -16 * ONE)


def test_matvec_fixed_reference_kats():
    # engine/tests.rs:389-407: 2x2 Q8_0, d = 0.5, codes 3 and 2, x = [1, 1] -> y = [2, 1].
    raw = np.zeros(68, np.uint8)
    raw[0:2] = [0x00, 0x38]
    raw[34:36] = [0x00, 0x38]
    raw[2], raw[36] = 3, 2
    st, y = oracle.matvec_fixed(8, raw, 2, 2, [1, 1])
    assert st == 0 and y.tolist() == [2, 1]
    # engine/tests.rs:435-439 ties via a one-weight row of value ONE/2: 1.5 -> 2, -1.5 -> -1, 0.5 -> 1
    r1 = np.zeros(34, np.uint8)
    r1[0:2] = [0x00, 0x38]
    r1[2] = 1
    assert oracle.matvec_fixed(8, r1, 1, 1, [3])[1].tolist() == [2]
    assert oracle.matvec_fixed(8, r1, 1, 1, [-3])[1].tolist() == [-1]
    assert oracle.matvec_fixed(8, r1, 1, 1, [1])[1].tolist() == [1]
    # engine/tests.rs:409-432 refusals
    assert oracle.matvec_fixed(8, np.zeros(68, np.uint8), 2, 2, [ONE])[0] == 1
    assert oracle.matvec_fixed(8, np.zeros(34, np.uint8), 2, 2, [ONE, ONE])[0] == 3
    assert oracle.matvec_fixed(999, np.zeros(4, np.uint8), 1, 1, [ONE])[0] == 5


# families the CPU baseline's fast cores cover (the benchmarked ones); Q2_K and Q3_K have the
# contract only
FAST_TYPES = (6, 8, 12, 14)

SHAPES = [(4, 32), (3, 48), (2, 33), (2, 300), (1, 64), (5, 0), (1, 256), (2, 512), (2, 256)]


@pytest.mark.parametrize("t", [6, 8, 10, 11, 12, 14])
def test_matvec_random_payloads_vs_bruteforce(t):
    # chart/tests.rs:222-267 shapes, random block bytes with d = dmin = 0x3800.
    rng = np.random.default_rng(0x12345678 + t)
    for rows, n_in in SHAPES + [(2, w) for w in (33, 47, 65, 257, 300, 271)]:
        raw = synth.random_bytes_payload(rng, t, rows, n_in, 0x3800, 0x3800)
        x = (rng.integers(0, 4096, size=n_in) - 2048).astype(np.int64)
        st, codes, scales = oracle.quant_act(x)
        assert st == 0
        st, y = oracle.matvec_q8act(t, raw, rows, n_in, codes, scales)
        xhat = oracle.dequant_act(codes, scales)[1]
        want = bf.matvec(t, raw.tobytes(), rows, n_in, xhat.tolist())
        assert st == 0 and y.tolist() == want, (t, rows, n_in)
        if t in FAST_TYPES:
            stf, yf = oracle.matvec_q8act_fast(t, raw, rows, n_in, codes, scales, 2)
            assert stf == 0 and yf.tolist() == want, (t, rows, n_in)
        # the tolerance basis sum_i |w_i * xhat_i| (real units) against exact integers
        sta, absdot = oracle.row_absdot(t, raw, rows, n_in, codes, scales)
        assert sta == 0
        for r in range(rows):
            rb = synth.row_bytes(t, n_in)
            row = raw[r * rb:(r + 1) * rb]
            wq = bf.weights_row(t, row.tobytes(), n_in)
            exact = sum(abs(wi * xi) for wi, xi in zip(wq, xhat.tolist())) / 2.0 ** 64
            assert abs(absdot[r] - exact) <= 1e-12 * exact, (t, rows, n_in, r)
            st, dots, xs = oracle.block_dots(t, row, n_in, codes)
            assert st == 0
            assert dots.tolist() == bf.block_dots(t, row.tobytes(), n_in, codes.tolist())
            assert xs.tolist() == [int(codes[b:b + 32].astype(np.int64).sum()) for b in range(0, n_in, 32)]


@pytest.mark.parametrize("t", [6, 8, 10, 11, 12, 14])
def test_extreme_scales_and_codes(t):
    # chart/tests.rs:269-307: largest finite scale 0x7BFF, codes +-127 at unit scale.
    rng = np.random.default_rng(0x51FF0000 + t)
    raw = synth.random_bytes_payload(rng, t, 2, 256, 0x7BFF, 0x7BFF)
    codes = np.array([127 if j % 2 == 0 else -127 for j in range(256)], np.int8)
    scales = np.ones(8, np.int64)
    st, y = oracle.matvec_q8act(t, raw, 2, 256, codes, scales)
    want = bf.matvec(t, raw.tobytes(), 2, 256, [int(c) for c in codes])
    assert st == 0 and y.tolist() == want
    if t in FAST_TYPES:
        assert oracle.matvec_q8act_fast(t, raw, 2, 256, codes, scales, 1)[1].tolist() == want


def test_q2_k_q3_k_unpack_kats():
    # format/quant.rs:811-822: qs byte 16 = 0b11_10_01_00 carries outputs 0, 32, 64, 96 (one bit
    # pair each, consecutive pairs 32 outputs apart); output 16 (the next plane) is 0.  Read
    # through the dequantizer with d = 1.0, dmin = 0 and every group scale 1, so w = q.
    b2 = np.zeros(84, np.uint8)
    b2[0:16] = 0x01
    b2[16] = 0b11_10_01_00
    b2[80:82] = [0x00, 0x3C]
    st, w = oracle.dequant_row(10, b2, 256)
    assert st == 0
    assert [int(w[i]) // ONE for i in (0, 32, 64, 96, 16)] == [0, 1, 2, 3, 0]
    # format/quant.rs:859-869: scale byte 0x51 is (scale 1, min 5); d = 1.0 at byte 80, dmin = 0.5
    # at byte 82 -- so group 0 holds w = q - 2.5 and every other (zero) group w = 0
    b2 = np.zeros(84, np.uint8)
    b2[0] = 0x51
    b2[16] = 0b11_10_01_11
    b2[80:84] = [0x00, 0x3C, 0x00, 0x38]
    st, w = oracle.dequant_row(10, b2, 256)
    assert st == 0
    assert int(w[0]) == 3 * ONE - 5 * ONE // 2 and int(w[1]) == -5 * ONE // 2 and int(w[16]) == 0
    # format/quant.rs:870-872: Q3_K's d sits at byte 108.  All other bytes zero: every 6-bit scale
    # 0 (factor 0 - 32) and every hmask bit clear (code 0 - 4), so w = 1.0 * -32 * -4 = 128
    b3 = np.zeros(110, np.uint8)
    b3[108:110] = [0x00, 0x3C]
    st, w = oracle.dequant_row(11, b3, 256)
    assert st == 0 and set((w // ONE).tolist()) == {128}
    # Q3_K's scale shuffle (format/quant.rs:391-417): groups whose 6-bit scale is 32 + j for j in
    # 0..15, packed positionally (low nibbles in bytes 0..7, high bit pairs in bytes 8..11); all
    # hmask bits set and qs bits 1, so every code is 1 and w = j in group j
    want = [32 + j for j in range(16)]
    b3 = np.zeros(110, np.uint8)
    b3[0:32] = 0xFF
    b3[32:96] = 0b01010101
    for j, v in enumerate(want):
        if j < 8:
            b3[96 + j] |= v & 0xF
        else:
            b3[96 + j - 8] |= (v & 0xF) << 4
        b3[104 + j % 4] |= ((v >> 4) & 3) << (2 * (j // 4))
    b3[108:110] = [0x00, 0x3C]
    assert bf.q3k_scales(bytes(b3[96:108])) == want
    st, w = oracle.dequant_row(11, b3, 256)
    assert st == 0 and (w // ONE).tolist() == [e // 16 for e in range(256)]
    # every (qs bit pair, hmask bit) position: one set bit at a time against the brute force
    for byte in range(96):
        for bit in range(8):
            b3 = np.zeros(110, np.uint8)
            b3[96:108] = rng_bytes(byte * 8 + bit)
            b3[108:110] = [0x00, 0x3C]
            b3[byte] = 1 << bit
            st, w = oracle.dequant_row(11, b3, 256)
            assert st == 0 and w.tolist() == bf.weights_row(11, bytes(b3), 256)
            b2 = np.zeros(84, np.uint8)
            b2[0:16] = rng_bytes(byte * 8 + bit)[:12].tolist() + [0x21, 0x43, 0x65, 0x87]
            b2[80:84] = [0x00, 0x3C, 0x00, 0x34]
            if 16 <= byte < 80:
                b2[byte] = 1 << bit
            st, w = oracle.dequant_row(10, b2, 256)
            assert st == 0 and w.tolist() == bf.weights_row(10, bytes(b2), 256)


def rng_bytes(seed):
    return np.random.default_rng(seed).integers(0, 256, size=12, dtype=np.uint8)


def test_q8_0_scale_sets_and_spread(cpu_path):
    # kern/gemm.rs:2613-2617 scale-word sets (subnormal, negative, zero, largest) and wide
    # activation spreads (kern/gemm.rs:2490-2506).
    sets = [[0x2000, 0x2400, 0x1C00, 0xA000], [0x0001, 0x03FF, 0x0400, 0x8200],
            [0x0000, 0x3C00, 0x0010, 0x7BFF]]
    rng = np.random.default_rng(0x6E6D6D71)
    for si, words in enumerate(sets):
        for rng_bits in (1, 8, 30):
            n_out, n_in = 5, 96
            raw = rng.integers(0, 256, size=(n_out * 3, 34), dtype=np.uint8)
            w = rng.choice(words, size=n_out * 3)
            raw[:, 0], raw[:, 1] = w & 0xFF, w >> 8
            raw = raw.reshape(-1)
            mags = 1 << (20 + rng.integers(0, rng_bits, size=n_in))
            x = np.array([int(rng.integers(-m, m + 1)) if (j // 32) % 7 != 3 else 0
                          for j, m in enumerate(mags.tolist())], dtype=np.int64)
            st, codes, scales = oracle.quant_act(x)
            assert st == 0
            xhat = oracle.dequant_act(codes, scales)[1]
            want = bf.matvec(8, raw.tobytes(), n_out, n_in, xhat.tolist())
            st, y = oracle.matvec_q8act(8, raw, n_out, n_in, codes, scales)
            stf, yf = oracle.matvec_q8act_fast(8, raw, n_out, n_in, codes, scales, 3)
            if any(not I64_MIN <= v <= I64_MAX for v in want):
                # the contract refuses an output that leaves i64 (ops/matvec.rs:113-115)
                assert st == 9 and stf == 9, (si, rng_bits)
                continue
            assert st == 0 and y.tolist() == want, (si, rng_bits)
            assert stf == 0 and yf.tolist() == want


def test_nonfinite_scale_refuses(cpu_path):
    # kern/gemm.rs:2756-2763: an f16 +inf scale refuses (NonFiniteScale), also on the fast path
    # (every core form: the bad scale sits in the second row, i.e. in a two-row tile).
    rng = np.random.default_rng(1)
    for t in (8, 10, 11, 12, 14):
        raw = synth.random_bytes_payload(rng, t, 3, 256, 0x3800, 0x3800)
        rb = synth.row_bytes(t, 256)
        od, om = synth.SCALE_AT[t]
        off = rb + (om if om is not None else od)  # Q2_K / Q4_K: the dmin word
        raw[off:off + 2] = [0x00, 0x7C]
        st, codes, scales = oracle.quant_act(np.arange(256, dtype=np.int64) - 100)
        assert oracle.matvec_q8act(t, raw, 3, 256, codes, scales)[0] == 6
        if t in FAST_TYPES:
            assert oracle.matvec_q8act_fast(t, raw, 3, 256, codes, scales, 2)[0] == 6


def test_zero_activation_blocks():
    # chart/tests.rs:336-371
    x = np.zeros(96, np.int64)
    x[64:] = 1000 - 100 * np.arange(64, 96)
    st, codes, scales = oracle.quant_act(x)
    assert st == 0 and not codes[:64].any() and scales[0] == 0 and scales[1] == 0
    rng = np.random.default_rng(0x9000)
    for t in (8, 12, 14):
        raw = synth.random_bytes_payload(rng, t, 1, 96, 0x3800, 0x3800)
        xhat = oracle.dequant_act(codes, scales)[1]
        want = bf.matvec(t, raw.tobytes(), 1, 96, xhat.tolist())
        assert oracle.matvec_q8act(t, raw, 1, 96, codes, scales)[1].tolist() == want


def test_matmat_fast_equals_per_column_contract(cpu_path):
    # kern/matmat.rs:973-1149 shape: every column equals the per-column contract.
    rng = np.random.default_rng(21)
    for t, n_out, n_in in [(8, 17, 64), (12, 9, 512), (14, 7, 256), (12, 5, 896), (8, 3, 96), (6, 11, 96),
                           (6, 4, 896)]:
        raw = synth.payload(t, rng, n_out, n_in)
        x = synth.activations(rng, n_in, 9)
        st, codes, scales = oracle.quant_act_f32_batch(x)
        assert st == 0
        st, y = oracle.matmat_q8act_fast(t, raw, n_out, n_in, codes, scales, 3)
        assert st == 0
        for c in range(9):
            assert y[c].tolist() == oracle.matvec_q8act(t, raw, n_out, n_in, codes[c], scales[c])[1].tolist()


def test_q5_0_every_code_and_bit_position():
    # Each of the 32 outputs takes its nibble and its qh bit from the position the layout fixes:
    # a block whose only nonzero field is one nibble or one qh bit changes exactly one output.
    for e in range(32):
        for field in ("nib", "bit"):
            b5 = np.zeros(22, np.uint8)
            b5[0:2] = [0x00, 0x3C]  # d = 1
            if field == "nib":
                b5[6 + e % 16] = 0x0F if e < 16 else 0xF0
            else:
                b5[2 + e // 8] = 1 << (e % 8)
            w = oracle.dequant_row(6, b5, 32)[1] // ONE
            want = [-16] * 32
            want[e] = -1 if field == "nib" else 0
            assert w.tolist() == want, (e, field)
            assert bf.q5_0_codes(bytes(b5)) == want


def test_synth_generators_roundtrip():
    # The packers invert the reference unpack rules (format/quant.rs:482-491, :574-599).
    rng = np.random.default_rng(4)
    sc = rng.integers(0, 64, size=(50, 8))
    m = rng.integers(0, 64, size=(50, 8))
    packed = synth.pack_q4_k_scales(sc, m)
    for i in range(50):
        assert bf.q4k_pairs(bytes(packed[i])) == list(zip(sc[i].tolist(), m[i].tolist()))
    u = rng.integers(0, 64, size=(3, 256))
    ql, qh = synth.pack_q6_k_codes(u)
    for i in range(3):
        blk = np.zeros(210, np.uint8)
        blk[:128], blk[128:192] = ql[i], qh[i]
        blk[192:208] = 1
        blk[208:210] = [0x00, 0x3C]
        w = oracle.dequant_row(14, blk, 256)[1]
        assert (w // ONE + 32).tolist() == u[i].tolist()


@pytest.fixture(params=[oracle.CPU_PORTABLE, oracle.CPU_AVX2, oracle.CPU_VNNI], ids=["portable", "avx2", "vnni"])
def cpu_path(request):
    """Each core form of the fast CPU path the host offers (skipped where the host lacks it)."""
    got = oracle.set_cpu_path(request.param)
    try:
        if got != request.param:
            pytest.skip("the host lacks this core form")
        yield got
    finally:
        oracle.set_cpu_path(-1)


@pytest.mark.parametrize("t", [6, 8, 12, 14])
def test_fast_cores_equal_contract(t, cpu_path):
    """Every core form (portable, AVX2 maddubs, AVX-VNNI vpdpbusd; rows one at a time or in the
    two-row tiles of x86.rs:782-1192) equals the exact contract, on odd and even row counts (a
    trailing single row after the pairs), ragged K, zero blocks and the reference's extreme scales,
    for the GEMV and for every column of the GEMM."""
    rng = np.random.default_rng(0xC0DE + t)
    for n_out, n_in in [(1, 256), (2, 96), (7, 512), (8, 896), (5, 300), (9, 1536)]:
        raw = synth.random_bytes_payload(rng, t, n_out, n_in, 0x3800, 0x2400)
        if t in (6, 8):  # the reference's scale words, including the largest and subnormal ones
            bb = 34 if t == 8 else 22
            words = rng.choice([0x0001, 0x03FF, 0x7BFF, 0x3C00, 0x0000, 0x8200], size=len(raw) // bb)
            blocks = raw.reshape(-1, bb)
            blocks[:, 0], blocks[:, 1] = words & 0xFF, words >> 8
        x = synth.activations(rng, n_in, 5)
        x[1, : min(64, n_in)] = 0.0  # zero blocks
        st, codes, scales = oracle.quant_act_f32_batch(x)
        assert st == 0
        want = []
        for c in range(5):
            stc, yc = oracle.matvec_q8act(t, raw, n_out, n_in, codes[c], scales[c])
            want.append((stc, yc.tolist()))
            stf, yf = oracle.matvec_q8act_fast(t, raw, n_out, n_in, codes[c], scales[c], 3)
            assert stf == stc, (t, n_out, n_in, c)
            if stc == 0:
                assert yf.tolist() == yc.tolist(), (t, n_out, n_in, c)
        if all(w[0] == 0 for w in want):
            st, y = oracle.matmat_q8act_fast(t, raw, n_out, n_in, codes, scales, 3)
            assert st == 0
            assert [y[c].tolist() for c in range(5)] == [w[1] for w in want], (t, n_out, n_in)
