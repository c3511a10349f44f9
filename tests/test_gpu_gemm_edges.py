"""GPU parity of the prefill GEMM on the reference's own edge-case inputs, through the C ABI.

The inputs follow the reference's GEMM equality tests, regenerated here with numpy (the
reference's LCG stream is not needed: the distributions are what the tests exercise):

* kern/gemm.rs:2607-2645 ``gemm_equals_the_per_column_contract``: Q8_0 payloads of random bytes
  (every code -128..127) whose block scales come from three scale-word sets (subnormal, zero,
  negative and the largest finite f16 among them), shapes (1,32) (17,64) (33,1024) (40,3584),
  k in {1,2,7,8,9,17,64} columns whose 32-blocks span 1, 8 or 30 bits of magnitude (2^20 ..
  2^49 in Q32.32) with every 7th block zero.  Wide spans drive some of those columns past the f16
  operand's band; the contract also refuses some calls with OutputOverflow.
* chart/tests.rs:1080-1110 ``spread_columns``: base values in [-2048, 2047] with block b shifted
  left by 29*b/(groups-1), for Q4_K / Q6_K / Q8_0 at n_out = 7, n_in in {256, 1024}.
* tests/golden/golden.npz: every fixture through the GEMM.
* A token whose largest blocks meet zero weights while the row's weight sits on blocks 2^27
  lower: under a per-token f16 band those blocks would be lost (the whole result), so the operand
  pass must route the token to the exact path.
* chart/tests.rs:525-560 ``chart_agrees_with_fixed_on_every_refusal_class``: each refusal class
  through the GPU forms.

Bar: every non-refused output within 1e-4 * sum|w*xhat| + 2^-32 of the oracle's exact value; the
call's status equal to the contract's first refusal (column, then row), except where an output
lies within that tolerance of the refusal bound (the f32 result cannot decide those).
"""
import os

import numpy as np
import pytest

import oracle
from apeiron_amd import chart, synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
TOL = 1e-4
Q32 = 2.0 ** -32
SCALE_SETS = ([0x2000, 0x2400, 0x1C00, 0xA000], [0x0001, 0x03FF, 0x0400, 0x8200],
              [0x0000, 0x3C00, 0x0010, 0x7BFF])


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    d = chart.Device(0)
    yield d
    d.close()


def stream():
    return torch.cuda.current_stream().cuda_stream


def to_dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


# ---- input generators (shapes and distributions of the reference tests) -------------------

def ref_q8_payload(rng, n_out, n_in, words):
    """kern/gemm.rs:2478-2489: per block a scale word from `words`, then 32 random bytes."""
    nb = n_out * (n_in // 32)
    blk = rng.integers(0, 256, size=(nb, 34), dtype=np.uint8)
    w = np.asarray(words, np.uint16)[rng.integers(0, len(words), size=nb)]
    blk[:, 0], blk[:, 1] = w & 0xFF, w >> 8
    return blk.reshape(-1)


def ref_columns(rng, k, n_in, rng_bits):
    """kern/gemm.rs:2492-2506: Q32.32 columns, every 7th 32-block zero, magnitudes 2^(20+r)."""
    mag = np.left_shift(np.int64(1), 20 + rng.integers(0, max(rng_bits, 1), size=(k, n_in)))
    x = rng.integers(-mag, mag + 1)
    x[:, (np.arange(n_in) // 32) % 7 == 3] = 0
    return x.astype(np.int64)


def spread_columns(rng, n_in, k):
    """chart/tests.rs:1080-1110: block b of a [-2048, 2047] column shifted by 29*b/(groups-1)."""
    groups = n_in // 32
    x = rng.integers(-2048, 2048, size=(k, n_in)).astype(np.int64)
    for b in range(groups):
        x[:, 32 * b:32 * b + 32] <<= (b * 29) // (groups - 1) if groups > 1 else 0
    return x


def quantize(x2d):
    k, n_in = x2d.shape
    nb = -(-n_in // 32)
    codes = np.zeros((k, n_in), np.int8)
    scales = np.zeros((k, nb), np.int64)
    for c in range(k):
        st, codes[c], scales[c] = oracle.quant_act(x2d[c])
        assert st == 0
    return codes, scales


# ---- GPU calls -------------------------------------------------------------------------------

def gemm_codes(dev, w, codes, scales):
    assert codes.ndim == 2 and codes.shape[1] == w.n_in and scales.shape == (codes.shape[0], -(-w.n_in // 32))
    n_tok = codes.shape[0]
    dc, ds = to_dev(codes), to_dev(scales)
    y = torch.full((n_tok, max(w.n_out, 1)), float("nan"), dtype=torch.float32, device="cuda")
    w.gemm_q8_dev(dc.data_ptr(), ds.data_ptr(), n_tok, y.data_ptr(), stream())
    st = dev.sync_status(stream())
    return st, y.cpu().numpy()[:, :w.n_out]


def gemv_codes(dev, w, codes, scales):
    dc, ds = to_dev(codes), to_dev(scales)
    y = torch.full((max(w.n_out, 1),), float("nan"), dtype=torch.float32, device="cuda")
    w.gemv_q8_dev(dc.data_ptr(), ds.data_ptr(), y.data_ptr(), stream())
    st = dev.sync_status(stream())
    return st, y.cpu().numpy()[:w.n_out]


def gemm_f32(dev, w, x2d):
    # the library reads n_tok x n_in floats from the device copy: shapes are checked here
    assert x2d.ndim == 2 and x2d.shape[1] == w.n_in, x2d.shape
    n_tok = x2d.shape[0]
    dx = to_dev(x2d.astype(np.float32))
    y = torch.full((n_tok, max(w.n_out, 1)), float("nan"), dtype=torch.float32, device="cuda")
    w.gemm_f32_dev(dx.data_ptr(), n_tok, y.data_ptr(), stream())
    st = dev.sync_status(stream())
    return st, y.cpu().numpy()[:, :w.n_out]


# ---- the contract, per row -------------------------------------------------------------------

def row_values_f64(t, raw, n_out, n_in, codes, scales):
    """Each row's real value in float64 from the exact Q32.32 weights and activation (used only to
    tell how far a refused or refusable output lies from the refusal bound)."""
    rb = synth.row_bytes(t, n_in)
    st, xh = oracle.dequant_act(codes, scales)
    assert st == 0
    xr = xh.astype(np.float64) * Q32
    out = np.zeros(n_out)
    for r in range(n_out):
        st, w = oracle.dequant_row(t, raw[r * rb:(r + 1) * rb], n_in)
        assert st == 0
        out[r] = float(np.dot(w.astype(np.float64) * Q32, xr))
    return out


def check_call(t, raw, n_out, n_in, codes, scales, st_gpu, Y, what):
    """Values of every column before the contract's first refusal within tolerance; the GPU status
    equal to that refusal's code unless an output it depends on is within tolerance of 2^31."""
    want_code, ambiguous = 0, False
    for c in range(codes.shape[0]):
        st, yref = oracle.matvec_q8act(t, raw, n_out, n_in, codes[c], scales[c])
        st2, absdot = oracle.row_absdot(t, raw, n_out, n_in, codes[c], scales[c])
        assert st2 == 0
        near = np.zeros(n_out, bool)
        if st or np.abs(yref).max(initial=0) * Q32 > 2.0 ** 30:
            yv = row_values_f64(t, raw, n_out, n_in, codes[c], scales[c])
            near = np.abs(np.abs(yv) - 2.0 ** 31) <= 2 * TOL * absdot + 1.0
        if st == 0:
            ref = yref.astype(np.float64) * Q32
            err = np.abs(Y[c].astype(np.float64) - ref)
            bad = np.nonzero(err > TOL * absdot + Q32)[0]
            assert bad.size == 0, f"{what} col {c}: rows {bad[:6]} err {err[bad[:6]]} tol {(TOL * absdot)[bad[:6]]}"
            ambiguous |= bool(near.any())
            continue
        assert st in (8, 9), (what, c, st)
        first = int(np.nonzero(np.abs(yv) >= 2.0 ** 31)[0][0]) if (np.abs(yv) >= 2.0 ** 31).any() else 0
        ambiguous |= bool(near[:first + 1].any())
        want_code = st
        break
    if not ambiguous:
        assert st_gpu == want_code, f"{what}: GPU status {st_gpu}, contract {want_code}"
    else:
        assert st_gpu in (0, want_code, 9), f"{what}: GPU status {st_gpu}"


# ---- tests -----------------------------------------------------------------------------------

@pytest.mark.parametrize("n_out,n_in", [(1, 32), (17, 64), (33, 1024), (40, 3584)])
def test_gemm_reference_equality_inputs(dev, n_out, n_in):
    """kern/gemm.rs:2607-2645 on the GPU GEMM (codes input), with GEMM(N=1) = GEMV on each."""
    rng = np.random.default_rng(0x6E6D6D71 + n_in)
    refusals = 0
    for k in (1, 2, 7, 8, 9, 17, 64):
        for si, words in enumerate(SCALE_SETS):
            for bits in (1, 8, 30):
                raw = ref_q8_payload(rng, n_out, n_in, words)
                codes, scales = quantize(ref_columns(rng, k, n_in, bits))
                w = dev.upload(8, raw, n_out, n_in)
                st, Y = gemm_codes(dev, w, codes, scales)
                what = f"{n_out}x{n_in} k{k} set{si} bits{bits}"
                check_call(8, raw, n_out, n_in, codes, scales, st, Y, what)
                refusals += st != 0
                if k == 1:
                    stv, yv = gemv_codes(dev, w, codes[0], scales[0])
                    check_call(8, raw, n_out, n_in, codes, scales, stv, yv[None, :], what + " gemv")
                w.free()
    if n_in >= 1024:
        assert refusals > 0  # the largest scale word drives some calls past 2^31


@pytest.mark.parametrize("t", [12, 14, 8, 6])
@pytest.mark.parametrize("n_in", [256, 1024])
def test_gemm_spread_columns(dev, t, n_in):
    """chart/tests.rs:1080-1110 (29 binades across a column) through the GEMM, n_out = 7."""
    rng = np.random.default_rng(0x5EED0A4B + t + n_in)
    raw = synth.payload(t, rng, 7, n_in)
    w = dev.upload(t, raw, 7, n_in)
    for k in (1, 3, 8, 9, 33):
        codes, scales = quantize(spread_columns(rng, n_in, k))
        st, Y = gemm_codes(dev, w, codes, scales)
        check_call(t, raw, 7, n_in, codes, scales, st, Y, f"spread t{t} K{n_in} k{k}")
    w.free()


def test_gemm_golden_fixtures(dev):
    """Every golden fixture as a GEMM: its column, a zero column and its column again."""
    z = np.load(GOLDEN, allow_pickle=False)
    n = 0
    for i in range(int(z["count"])):
        p = f"c{i:03d}_"
        t, rows, n_in = (int(v) for v in z[p + "meta"])
        raw, codes, scales = z[p + "raw"], z[p + "codes"], z[p + "scales"]
        w = dev.upload(t, raw, rows, n_in)
        C = np.stack([codes, np.zeros_like(codes), codes])
        S = np.stack([scales, np.zeros_like(scales), scales])
        st, Y = gemm_codes(dev, w, C, S)
        assert st == 0
        st2, absdot = oracle.row_absdot(t, raw, rows, n_in, codes, scales)
        ref = z[p + "y"].astype(np.float64) * Q32
        for c in (0, 2):
            err = np.abs(Y[c].astype(np.float64) - ref)
            assert (err <= TOL * absdot + Q32).all(), (str(z[p + "kind"]), t, n_in, c, err, absdot)
        assert (Y[1] == 0).all()
        if p + "xf" in z:
            xf = z[p + "xf"]
            stf, Yf = gemm_f32(dev, w, np.stack([xf, xf]))
            assert stf == 0
            for c in (0, 1):
                assert (np.abs(Yf[c].astype(np.float64) - ref) <= TOL * absdot + Q32).all()
        w.free()
        n += 1
    assert n >= 40


def cliff_case(t, n_in, gap, rng):
    """A payload whose first half of the row has zero weight scales and an activation whose first
    half sits 2^gap above the second: the whole result comes from the small blocks."""
    raw = synth.payload(t, rng, 16, n_in).copy()
    rb = synth.row_bytes(t, n_in)
    R = raw.reshape(16, rb)
    half = n_in // 2
    if t in (8, 6):
        bb = 34 if t == 8 else 22
        for b in range(half // 32):
            R[:, bb * b:bb * b + 2] = 0
    else:
        for sb in range(half // 256):
            off = (210 * sb + 208) if t == 14 else 144 * sb
            R[:, off:off + (2 if t == 14 else 4)] = 0  # d (and dmin): the super-block weighs 0
    x = rng.integers(-2048, 2048, size=(3, n_in)).astype(np.int64)
    x[:, :half] <<= gap
    x[1, :half] = 0  # a second token without the spread
    return R.reshape(-1), x


@pytest.mark.parametrize("t", [6, 8, 12, 14])
@pytest.mark.parametrize("gap", [27, 24, 20, 12])
def test_gemm_zero_weight_heavy_blocks(dev, t, gap):
    """Heavy blocks against zero weights, the rest 2^gap lower.  gap 27 is past the f16 band
    (the token takes the exact path); gap 24 and 20 keep it on the MFMA with subnormal f16
    operands (exact at 2^-24 and above); the GEMM equals the oracle and the GEMV either way."""
    rng = np.random.default_rng(1000 * t + gap)
    n_in = 1024
    raw, x = cliff_case(t, n_in, gap, rng)
    codes, scales = quantize(x)
    w = dev.upload(t, raw, 16, n_in)
    st, Y = gemm_codes(dev, w, codes, scales)
    check_call(t, raw, 16, n_in, codes, scales, st, Y, f"cliff t{t} gap{gap}")
    for c in range(3):
        stv, yv = gemv_codes(dev, w, codes[c], scales[c])
        check_call(t, raw, 16, n_in, codes[c:c + 1], scales[c:c + 1], stv, yv[None, :], f"cliff gemv t{t} c{c}")
    # one column alone (N = 1) on the GEMM as well
    st1, Y1 = gemm_codes(dev, w, codes[:1], scales[:1])
    check_call(t, raw, 16, n_in, codes[:1], scales[:1], st1, Y1, f"cliff N1 t{t}")
    w.free()


@pytest.mark.parametrize("t", [6, 8, 12, 14])
def test_gemm_f32_input_wide_spread_tokens(dev, t):
    """f32 input whose blocks span ~40 binades (flagged by the operand pass, whose quantized codes
    it keeps for the exact path) mixed with ordinary tokens, at a split-K shape and a small one."""
    rng = np.random.default_rng(77 + t)
    for n_out, n_in, n_tok in ((1536, 8960, 70), (96, 512, 9)):
        raw = synth.payload(t, rng, n_out, n_in)
        x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
        nb = n_in // 32
        for tok in range(0, n_tok, 3):  # every third token spread: block b times 2^(40 b / nb - 20)
            x[tok] *= np.repeat(np.exp2(np.arange(nb) * 40.0 / nb - 20.0), 32).astype(np.float32)
        w = dev.upload(t, raw, n_out, n_in)
        st, Y = gemm_f32(dev, w, x)
        assert st == 0
        rows = np.unique(rng.integers(0, n_out, 48))
        rb = synth.row_bytes(t, n_in)
        sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
        for c in range(n_tok):
            sto, codes, scales = oracle.quant_act_f32(x[c])
            assert sto == 0
            st1, yref = oracle.matvec_q8act(t, sub, len(rows), n_in, codes, scales)
            st2, absdot = oracle.row_absdot(t, sub, len(rows), n_in, codes, scales)
            err = np.abs(Y[c, rows].astype(np.float64) - yref.astype(np.float64) * Q32)
            assert (err <= TOL * absdot + Q32).all(), (t, n_out, n_in, c, err.max())
        w.free()


@pytest.mark.parametrize("t", [6, 8, 10, 11, 12, 14])
def test_gemm_exact_path_every_row_to_the_payload_end(dev, t):
    """Flagged tokens (blocks spanning 40 binades, past the f16 band) checked at every row, the
    last included: the exact path reads each weight unit from memory, and a unit within 16 bytes
    of the payload's end takes the byte-exact row form instead.  Twenty flagged tokens, more than
    one batch (8) per token tile, on an uploaded payload (its device size is the payload's) and on
    a wrapped one of exactly the payload's bytes."""
    rng = np.random.default_rng(1234 + t)
    n_out, n_in, n_tok = 72, 1024, 40
    raw = synth.payload(t, rng, n_out, n_in)
    x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
    nb = n_in // 32
    spread = np.repeat(np.exp2(np.arange(nb) * 40.0 / nb - 20.0), 32).astype(np.float32)
    for tok in range(0, n_tok, 2):
        x[tok] *= spread
    ref = []
    for c in range(n_tok):
        sto, codes, scales = oracle.quant_act_f32(x[c])
        assert sto == 0
        st1, yref = oracle.matvec_q8act(t, raw, n_out, n_in, codes, scales)
        st2, absdot = oracle.row_absdot(t, raw, n_out, n_in, codes, scales)
        assert st1 == 0 and st2 == 0
        ref.append((yref.astype(np.float64) * Q32, absdot))
    draw = to_dev(raw)
    for form in ("upload", "wrap"):
        if form == "upload":
            w = dev.upload(t, raw, n_out, n_in)
        else:
            w = dev.wrap(t, draw.data_ptr(), raw.nbytes, n_out, n_in)
        st, Y = gemm_f32(dev, w, x)
        assert st == 0, (t, form)
        for c, (yr, absdot) in enumerate(ref):
            err = np.abs(Y[c].astype(np.float64) - yr)
            assert (err <= TOL * absdot + Q32).all(), (t, form, c, int(np.argmax(err)), err.max())
        w.free()


def test_refusal_classes_match_reference(dev):
    """chart/tests.rs:525-560 through the GPU forms: each refusal class gives the contract's."""
    rng = np.random.default_rng(7)
    raw = synth.random_bytes_payload(rng, 8, 2, 32, 0x3800, 0x3800)
    x = rng.integers(-2048, 2048, size=32)
    q = dev.quant_act(x)
    import ctypes
    vp = ctypes.c_void_p
    # shape mismatch: the activation's length differs from n_in (ah_matvec_q8act's n_codes)
    w31 = dev.upload(8, raw, 2, 31)
    y2 = np.zeros(2, np.float32)
    st = dev.lib.ah_matvec_q8act(dev.h, w31.h, q.codes.ctypes.data_as(vp), q.scales.ctypes.data_as(vp),
                                 32, y2.ctypes.data_as(vp))
    assert st == 1
    w31.free()
    st, _ = oracle.matvec_q8act(8, raw, 2, 31, q.codes, q.scales)
    assert st == 1
    # short payload, unsupported family, row-stride overflow: refused at upload
    for args, code in (((8, raw[:-1], 2, 32), 3), ((0, raw[:0], 1, 1), 5)):
        with pytest.raises(chart.MatvecError) as e:
            dev.upload(*args)
        assert e.value.status == code
    h = ctypes.c_void_p()
    st = dev.lib.ah_upload_weight(dev.h, 8, raw.ctypes.data_as(ctypes.c_void_p), raw.nbytes,
                                  ctypes.c_size_t(2 ** 64 - 1), 32, ctypes.byref(h))
    assert st == 4
    # non-finite weight scale: NonFiniteScale { bits: 0x7C00 }
    inf = raw.copy()
    inf[0:2] = [0x00, 0x7C]
    with pytest.raises(chart.MatvecError) as e:
        dev.upload(8, inf, 2, 32)
    assert e.value.status == 6 and dev.last_refusal_bits() == 0x7C00
    dinf = to_dev(inf)
    with pytest.raises(chart.MatvecError) as e:
        dev.wrap(8, dinf.data_ptr(), inf.nbytes, 2, 32)
    assert e.value.status == 6 and dev.last_refusal_bits() == 0x7C00
    # output overflow: weight 1.0 against 127 * 2^56 (GEMV host form, GEMV and GEMM device forms)
    one = synth.random_bytes_payload(rng, 8, 1, 32, 0x3C00, 0x3800)
    one[2:34] = 1
    top = np.full(32, 127 << 56, np.int64)
    qt = dev.quant_act(top)
    assert (qt.codes == 127).all() and qt.scales.tolist() == [1 << 56]
    with pytest.raises(chart.MatvecError) as e:
        chart.matvec_q8act(8, one, 1, 32, qt)
    assert e.value.status == 9
    assert oracle.matvec_q8act(8, one, 1, 32, qt.codes, qt.scales)[0] == 9
    w1 = dev.upload(8, one, 1, 32)
    assert gemv_codes(dev, w1, qt.codes, qt.scales)[0] == 9
    C = np.stack([np.zeros(32, np.int8), qt.codes])
    S = np.stack([np.zeros(1, np.int64), qt.scales])
    assert gemm_codes(dev, w1, C, S)[0] == 9
    assert gemv_codes(dev, w1, np.zeros(32, np.int8), np.zeros(1, np.int64))[0] == 0  # cleared
    w1.free()
    # a QuantAct whose dequantized activation cannot exist: Dequant(FixedOverflow)
    w_1 = dev.upload(8, raw[:34], 1, 1)
    imp = chart.QuantAct(np.array([2 ** 63 - 1], np.int64), np.array([127], np.int8))
    with pytest.raises(chart.MatvecError) as e:
        chart.matvec_q8act(8, raw[:34], 1, 1, imp)
    assert e.value.status == 7
    assert oracle.matvec_q8act(8, raw[:34], 1, 1, imp.codes, imp.scales)[0] == 7
    w_1.free()


def test_gemm_odd_scale_quantacts(dev):
    """Hand-built QuantActs whose scales are not powers of two (any i64 the reference accepts that
    dequantizes): the GEMM serves them on the exact path and matches the GEMV and the contract."""
    rng = np.random.default_rng(11)
    for t in (8, 12, 14):
        n_out, n_in = 40, 512
        raw = synth.payload(t, rng, n_out, n_in)
        codes, scales = quantize(rng.integers(-4096, 4096, size=(4, n_in)).astype(np.int64))
        scales[1] = scales[1] * 3  # 3 * 2^e
        scales[2, ::2] = -scales[2, ::2]  # negative scales
        w = dev.upload(t, raw, n_out, n_in)
        st, Y = gemm_codes(dev, w, codes, scales)
        check_call(t, raw, n_out, n_in, codes, scales, st, Y, f"odd scales t{t}")
        w.free()


def big_k23_payload(t, n_out, n_in):
    """Every weight of every row the same sign and near the type's largest magnitude: Q2_K scale
    bytes 0xFF (sc = m = 15), codes 3, d = 65504, dmin = -65504 (w = 65504 * 60); Q3_K all-zero
    code, mask and scale bytes (sc - 32 = -32, q - 4 = -4) with d = 65504 (w = 65504 * 128)."""
    rb = synth.row_bytes(t, n_in)
    blk = np.zeros((n_out * (n_in // 256), rb // (n_in // 256)), np.uint8)
    if t == 10:
        blk[:, 0:80] = 0xFF
        blk[:, 80], blk[:, 81], blk[:, 82], blk[:, 83] = 0xFF, 0x7B, 0xFF, 0xFB
    else:
        blk[:, 108], blk[:, 109] = 0xFF, 0x7B
    return blk.reshape(-1)


@pytest.mark.parametrize("t", [10, 11])
@pytest.mark.parametrize("design", [0, 1])
def test_k23_refusal_order_across_tokens(dev, t, design):
    """The first refusal of a prefill is the first refusing column's (chart/mod.rs:1955-1975 runs
    matvec_q8act column by column), also when a later column refuses at an earlier row with a
    smaller code: OutputOverflow (9) of column 0 wins over AccumulatorOverflow (8) of column 1
    and the reverse.  Q2_K / Q3_K through the tiles (AUTO) and the per-token GEMV route (F16)."""
    n_out, n_in = 3, 4096
    raw = big_k23_payload(t, n_out, n_in)
    w = dev.upload(t, raw, n_out, n_in)
    dev.set_gemm_design(t, design)
    try:
        mid = (np.full(n_in, 127, np.int8), np.full(n_in // 32, 1 << 40, np.int64))  # |y| ~ 2^50
        top = (np.full(n_in, 127, np.int8), np.full(n_in // 32, 1 << 56, np.int64))   # |y| >= 2^63
        low = (np.full(n_in, 1, np.int8), np.full(n_in // 32, 1 << 20, np.int64))     # no refusal
        for c, want in (((mid, top), 9), ((top, mid), 8), ((low, mid), 9), ((low, top), 8),
                        ((low, low, top, mid, low), 8), ((low, low, low, low, mid, top), 9)):
            codes = np.stack([q[0] for q in c])
            scales = np.stack([q[1] for q in c])
            firsts = [oracle.matvec_q8act(t, raw, n_out, n_in, q[0], q[1])[0] for q in c]
            assert next(s for s in firsts if s) == want  # the contract, column by column
            st, _ = gemm_codes(dev, w, codes, scales)
            assert st == want, (t, design, firsts, st)
        # the same from f32 activations: 127 * 2^8 quantizes to codes 127 at scale 2^40, 2^30 to
        # codes 64 at scale 2^56 (|y| >= 2^63 still)
        xm = np.full(n_in, 127.0 * 256.0, np.float32)
        xt = np.full(n_in, 2.0 ** 30, np.float32)
        for rows, want in (((xm, xt), 9), ((xt, xm), 8)):
            st, _ = gemm_f32(dev, w, np.stack(rows))
            assert st == want, (t, design, st)
        # input refusals across tokens: token 0 out of range (InputRange, 11) at element 100, token 1
        # non-finite (NonFinite, 10) at element 0 -- the first token's refusal
        xr = np.full(n_in, 1.0, np.float32)
        xr[100] = 2.0 ** 32
        xn = np.full(n_in, 1.0, np.float32)
        xn[0] = np.nan
        for rows, want in (((xr, xn), 11), ((xn, xr), 10)):
            assert [oracle.quant_act_f32(r)[0] for r in rows][0] == want
            st, _ = gemm_f32(dev, w, np.stack(rows))
            assert st == want, (t, design, st)
    finally:
        dev.set_gemm_design(t, 0)
        w.free()
