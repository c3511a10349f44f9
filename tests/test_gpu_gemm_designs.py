"""The prefill GEMM designs of Q8_0 and Q4_K against the oracle on the same inputs, through the C ABI.

Q8_0 runs on the f16-MFMA design by default; ah_set_gemm_design selects the int8-MFMA design
(v_mfma_i32_32x32x32_i8 exact block dots, folded with d * 2^(e_b - E) from a bf16 outer-product
MFMA).  The edge-case suite (test_gpu_gemm_edges) runs the default; here:

* the int8 design repeats the Q8_0 edge cases (kern/gemm.rs:2607-2645 inputs, the golden
  fixtures, heavy blocks against zero weights at gaps past and inside the f16 band);
* both designs meet the oracle on the configs[3] Q8_0 shapes at N = 512 (sampled rows, every
  split-K form the host picks) and on ragged token counts;
* a grouped call of Q8_0 beside Q4_K / Q6_K parts (the operand pass writes both designs'
  operands at once) meets the oracle part by part;
* the int8 design keeps a token whose blocks span 50 binades on the MFMA (no f16 band): its
  result meets the oracle as the f16 design's exact path does.

Q4_K runs on the f16-MFMA design by default; its int8 design takes the exact sub-block dots of
the nibbles from the int8 MFMA and folds d sc_j and dmin m_j (split into three bf16 each) against
the token's block factor and its scaled code sum X_b (two bf16, written by the operand pass) with
bf16 outer-product MFMAs.  It repeats the edge cases that reach it (spread columns, the golden
fixtures, heavy blocks, odd-scale QuantActs on the exact path), the configs[4] shapes, ragged
token counts and a grouped call beside Q8_0 (int8) and Q6_K (f16) parts.

Bar: |y - y_ref| <= 1e-4 * sum|w*xhat| + 2^-32 per output (y_ref the exact Q32.32 contract).
"""
import numpy as np
import pytest

import oracle
from apeiron_amd import chart, synth
from test_gpu_gemm_edges import (SCALE_SETS, check_call, cliff_case, gemm_codes, gemm_f32, quantize,
                                 ref_columns, ref_q8_payload, spread_columns, GOLDEN)

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-4
Q32 = 2.0 ** -32
Q8_0, Q4_K, Q6_K = 8, 12, 14
F16, INT8 = chart.Device.GEMM_F16, chart.Device.GEMM_INT8


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    d = chart.Device(0)
    yield d
    d.close()


@pytest.fixture
def design(dev, request):
    dev.set_gemm_design(Q8_0, request.param)
    yield request.param
    dev.set_gemm_design(Q8_0, chart.Device.GEMM_AUTO)


def stream():
    return torch.cuda.current_stream().cuda_stream


def oracle_rows(t, raw, n_in, rows, x, y_rows, what):
    rb = synth.row_bytes(t, n_in)
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
    st, codes, scales = oracle.quant_act_f32(x)
    assert st == 0
    st, yref = oracle.matvec_q8act(t, sub, len(rows), n_in, codes, scales)
    st2, absdot = oracle.row_absdot(t, sub, len(rows), n_in, codes, scales)
    assert st == 0 and st2 == 0
    err = np.abs(np.asarray(y_rows, np.float64) - yref.astype(np.float64) * Q32)
    bad = np.nonzero(err > TOL * absdot + Q32)[0]
    assert bad.size == 0, f"{what}: rows {rows[bad[:6]]} err {err[bad[:6]]} tol {(TOL * absdot)[bad[:6]]}"


def test_design_selector_refusals(dev):
    """INT8 exists for Q8_0 and Q4_K only; unknown designs are invalid arguments."""
    dev.set_gemm_design(Q8_0, INT8)
    dev.set_gemm_design(Q8_0, F16)
    dev.set_gemm_design(Q4_K, INT8)
    dev.set_gemm_design(Q4_K, F16)
    with pytest.raises(chart.MatvecError):
        dev.set_gemm_design(Q6_K, INT8)
    with pytest.raises(chart.MatvecError):
        dev.set_gemm_design(Q8_0, 7)
    dev.set_gemm_design(Q8_0, chart.Device.GEMM_AUTO)
    dev.set_gemm_design(Q4_K, chart.Device.GEMM_AUTO)


@pytest.mark.parametrize("design", [INT8], indirect=True)
@pytest.mark.parametrize("n_out,n_in", [(17, 64), (40, 3584)])
def test_int8_design_reference_equality_inputs(dev, design, n_out, n_in):
    """kern/gemm.rs:2607-2645 inputs on the int8 design (codes input)."""
    rng = np.random.default_rng(0x6E6D0000 + n_in)
    for k in (1, 9, 64):
        for si, words in enumerate(SCALE_SETS):
            for bits in (1, 8, 30):
                raw = ref_q8_payload(rng, n_out, n_in, words)
                codes, scales = quantize(ref_columns(rng, k, n_in, bits))
                w = dev.upload(Q8_0, raw, n_out, n_in)
                st, Y = gemm_codes(dev, w, codes, scales)
                check_call(Q8_0, raw, n_out, n_in, codes, scales, st, Y, f"int8 {n_out}x{n_in} k{k} set{si} bits{bits}")
                w.free()


@pytest.mark.parametrize("design", [F16, INT8], indirect=True)
def test_designs_golden_fixtures_q8_0(dev, design):
    """Every Q8_0 golden fixture as a GEMM column on both designs."""
    z = np.load(GOLDEN, allow_pickle=False)
    n = 0
    for i in range(int(z["count"])):
        p = f"c{i:03d}_"
        t, rows, n_in = (int(v) for v in z[p + "meta"])
        if t != Q8_0:
            continue
        raw, codes, scales = z[p + "raw"], z[p + "codes"], z[p + "scales"]
        w = dev.upload(t, raw, rows, n_in)
        st, Y = gemm_codes(dev, w, np.stack([codes, codes]), np.stack([scales, scales]))
        assert st == 0
        st2, absdot = oracle.row_absdot(t, raw, rows, n_in, codes, scales)
        ref = z[p + "y"].astype(np.float64) * Q32
        for c in (0, 1):
            assert (np.abs(Y[c].astype(np.float64) - ref) <= TOL * absdot + Q32).all(), (str(z[p + "kind"]), c)
        w.free()
        n += 1
    assert n >= 10


@pytest.mark.parametrize("design", [F16, INT8], indirect=True)
@pytest.mark.parametrize("gap", [50, 27, 20])
def test_designs_zero_weight_heavy_blocks(dev, design, gap):
    """Heavy blocks against zero weights, the rest 2^gap lower (50 and 27: past the f16 band; the
    int8 design carries them on the MFMA, the f16 design on its exact path)."""
    rng = np.random.default_rng(5000 + gap)
    n_in = 1024
    raw, x = cliff_case(Q8_0, n_in, gap, rng)
    codes, scales = quantize(x)
    w = dev.upload(Q8_0, raw, 16, n_in)
    st, Y = gemm_codes(dev, w, codes, scales)
    check_call(Q8_0, raw, 16, n_in, codes, scales, st, Y, f"design {design} gap {gap}")
    w.free()


@pytest.mark.parametrize("design", [F16, INT8], indirect=True)
@pytest.mark.parametrize("n_out,n_in", [(4864, 896), (896, 4864), (8960, 1536), (1536, 8960)])
def test_designs_config3_q8_0_shapes(dev, design, n_out, n_in):
    """configs[3] Q8_0 shapes at N = 512 (f32 input): sampled rows of sampled tokens."""
    rng = synth.rng_for(3, 7000 + n_out + n_in)
    raw = synth.payload(Q8_0, rng, n_out, n_in)
    x = synth.activations(rng, n_in, 512)
    w = dev.upload(Q8_0, raw, n_out, n_in)
    st, Y = gemm_f32(dev, w, x)
    assert st == 0
    rows = np.concatenate([np.arange(4), np.unique(rng.integers(0, n_out, 60)), np.arange(n_out - 4, n_out)])
    for c in (0, 127, 128, 300, 511):
        oracle_rows(Q8_0, raw, n_in, rows, x[c], Y[c, rows], f"design {design} {n_out}x{n_in} col {c}")
    w.free()


@pytest.mark.parametrize("design", [F16, INT8], indirect=True)
@pytest.mark.parametrize("n_tok", [2, 129, 300])
def test_designs_ragged_tokens(dev, design, n_tok):
    """Token counts that leave partial 128-token tiles, every output row against the oracle."""
    rng = synth.rng_for(3, 7100 + n_tok)
    n_out, n_in = 200, 1216  # 38 blocks: a partial last stage of 4 blocks
    raw = synth.payload(Q8_0, rng, n_out, n_in)
    x = synth.activations(rng, n_in, n_tok)
    w = dev.upload(Q8_0, raw, n_out, n_in)
    st, Y = gemm_f32(dev, w, x)
    assert st == 0
    rows = np.arange(n_out)
    for c in sorted({0, n_tok // 2, n_tok - 1}):
        oracle_rows(Q8_0, raw, n_in, rows, x[c], Y[c], f"design {design} n_tok {n_tok} col {c}")
    w.free()


@pytest.mark.parametrize("design", [INT8], indirect=True)
def test_int8_design_beside_k_quant_parts(dev, design):
    """A grouped call of Q8_0, Q4_K and Q6_K parts on one input: one operand pass writes the int8
    codes for the Q8_0 part and the f16 operand for the others; each part against the oracle."""
    rng = synth.rng_for(3, 7200)
    n_in, n_tok = 1536, 160
    proj = [(Q8_0, 600), (Q4_K, 256), (Q6_K, 130), (Q8_0, 64)]
    raws = [synth.payload(t, rng, n, n_in) for t, n in proj]
    W = [dev.upload(t, r, n, n_in) for (t, n), r in zip(proj, raws)]
    x = synth.activations(rng, n_in, n_tok)
    dx = torch.from_numpy(x).cuda()
    ys = [torch.full((n_tok, n), float("nan"), dtype=torch.float32, device="cuda") for _, n in proj]
    chart.gemm_group_f32_dev(dev, W, dx.data_ptr(), n_tok, [y.data_ptr() for y in ys], stream())
    assert dev.sync_status(stream()) == 0
    for (t, n), raw, y in zip(proj, raws, ys):
        Y = y.cpu().numpy()
        rows = np.arange(n)
        for c in (0, 77, 159):
            oracle_rows(t, raw, n_in, rows, x[c], Y[c], f"group part t{t} n{n} col {c}")
    for w in W:
        w.free()


@pytest.fixture
def q4_design(dev, request):
    dev.set_gemm_design(Q4_K, request.param)
    yield request.param
    dev.set_gemm_design(Q4_K, chart.Device.GEMM_AUTO)


@pytest.mark.parametrize("q4_design", [INT8], indirect=True)
@pytest.mark.parametrize("n_in", [256, 1024])
def test_q4k_int8_spread_columns(dev, q4_design, n_in):
    """chart/tests.rs:1080-1110 (29 binades across a column), n_out = 7, codes input."""
    rng = np.random.default_rng(0x5EED0A4B + 12 + n_in)
    raw = synth.payload(Q4_K, rng, 7, n_in)
    w = dev.upload(Q4_K, raw, 7, n_in)
    for k in (1, 3, 8, 9, 33, 130):
        codes, scales = quantize(spread_columns(rng, n_in, k))
        st, Y = gemm_codes(dev, w, codes, scales)
        check_call(Q4_K, raw, 7, n_in, codes, scales, st, Y, f"int8 q4k spread K{n_in} k{k}")
    w.free()


@pytest.mark.parametrize("q4_design", [INT8], indirect=True)
def test_q4k_int8_golden_fixtures(dev, q4_design):
    """Every Q4_K golden fixture as a GEMM column (twice, a zero column between) on the int8 design."""
    z = np.load(GOLDEN, allow_pickle=False)
    n = 0
    for i in range(int(z["count"])):
        p = f"c{i:03d}_"
        t, rows, n_in = (int(v) for v in z[p + "meta"])
        if t != Q4_K:
            continue
        raw, codes, scales = z[p + "raw"], z[p + "codes"], z[p + "scales"]
        w = dev.upload(t, raw, rows, n_in)
        st, Y = gemm_codes(dev, w, np.stack([codes, np.zeros_like(codes), codes]),
                           np.stack([scales, np.zeros_like(scales), scales]))
        assert st == 0
        st2, absdot = oracle.row_absdot(t, raw, rows, n_in, codes, scales)
        ref = z[p + "y"].astype(np.float64) * Q32
        for c in (0, 2):
            assert (np.abs(Y[c].astype(np.float64) - ref) <= TOL * absdot + Q32).all(), (str(z[p + "kind"]), c)
        assert (Y[1] == 0).all()
        w.free()
        n += 1
    assert n >= 5


@pytest.mark.parametrize("q4_design", [INT8], indirect=True)
@pytest.mark.parametrize("gap", [50, 27, 20])
def test_q4k_int8_zero_weight_heavy_blocks(dev, q4_design, gap):
    """Heavy super-blocks against zero d and dmin, the rest 2^gap lower: carried on the MFMA (the
    bf16 block factors span the gap)."""
    rng = np.random.default_rng(6000 + gap)
    n_in = 1024
    raw, x = cliff_case(Q4_K, n_in, gap, rng)
    codes, scales = quantize(x)
    w = dev.upload(Q4_K, raw, 16, n_in)
    st, Y = gemm_codes(dev, w, codes, scales)
    check_call(Q4_K, raw, 16, n_in, codes, scales, st, Y, f"int8 q4k gap {gap}")
    w.free()


@pytest.mark.parametrize("q4_design", [INT8], indirect=True)
def test_q4k_int8_odd_scales_exact_path(dev, q4_design):
    """QuantActs whose scales are not powers of two (and negative ones) are flagged and served by
    the exact path from the int8 kernel's epilogue; ordinary tokens beside them stay on the MFMA."""
    rng = np.random.default_rng(12)
    n_out, n_in = 72, 1024
    raw = synth.payload(Q4_K, rng, n_out, n_in)
    codes, scales = quantize(rng.integers(-4096, 4096, size=(20, n_in)).astype(np.int64))
    scales[1::3] = scales[1::3] * 3
    scales[2::5, ::2] = -scales[2::5, ::2]
    w = dev.upload(Q4_K, raw, n_out, n_in)
    st, Y = gemm_codes(dev, w, codes, scales)
    check_call(Q4_K, raw, n_out, n_in, codes, scales, st, Y, "int8 q4k odd scales")
    w.free()


@pytest.mark.parametrize("q4_design", [INT8], indirect=True)
@pytest.mark.parametrize("n_out,n_in", [(8960, 1536), (1536, 8960), (4864, 896), (896, 4864)])
def test_q4k_int8_config_shapes(dev, q4_design, n_out, n_in):
    """configs[4]-sized Q4_K projections at N = 512 (f32 input; K = 896 ends in half a
    super-block): sampled rows of sampled tokens, every split-K form the host picks."""
    rng = synth.rng_for(4, 7300 + n_out + n_in)
    raw = synth.payload(Q4_K, rng, n_out, n_in)
    x = synth.activations(rng, n_in, 512)
    w = dev.upload(Q4_K, raw, n_out, n_in)
    st, Y = gemm_f32(dev, w, x)
    assert st == 0
    rows = np.concatenate([np.arange(4), np.unique(rng.integers(0, n_out, 60)), np.arange(n_out - 4, n_out)])
    for c in (0, 127, 128, 300, 511):
        oracle_rows(Q4_K, raw, n_in, rows, x[c], Y[c, rows], f"int8 q4k {n_out}x{n_in} col {c}")
    w.free()


@pytest.mark.parametrize("q4_design", [INT8], indirect=True)
@pytest.mark.parametrize("n_tok", [1, 129, 300])
def test_q4k_int8_ragged_tokens(dev, q4_design, n_tok):
    """Partial 128-token tiles and an odd stage count (K = 1280: 10 stages), every row."""
    rng = synth.rng_for(4, 7400 + n_tok)
    n_out, n_in = 200, 1280
    raw = synth.payload(Q4_K, rng, n_out, n_in)
    x = synth.activations(rng, n_in, n_tok).reshape(n_tok, n_in)  # one token: a 1-D draw
    w = dev.upload(Q4_K, raw, n_out, n_in)
    st, Y = gemm_f32(dev, w, x)
    assert st == 0
    for c in sorted({0, n_tok // 2, n_tok - 1}):
        oracle_rows(Q4_K, raw, n_in, np.arange(n_out), x[c], Y[c], f"int8 q4k n_tok {n_tok} col {c}")
    w.free()


@pytest.mark.parametrize("q4_design", [INT8], indirect=True)
def test_q4k_int8_beside_other_designs(dev, q4_design):
    """One grouped call: Q4_K parts on the int8 design, Q8_0 on the int8 design, Q6_K on the f16
    design; the operand pass writes the codes, block factors, scaled sums and the f16 operand at
    once and each part meets the oracle."""
    dev.set_gemm_design(Q8_0, INT8)
    try:
        rng = synth.rng_for(4, 7500)
        n_in, n_tok = 1536, 160
        proj = [(Q4_K, 600), (Q4_K, 256), (Q6_K, 130), (Q8_0, 64)]
        raws = [synth.payload(t, rng, n, n_in) for t, n in proj]
        W = [dev.upload(t, r, n, n_in) for (t, n), r in zip(proj, raws)]
        x = synth.activations(rng, n_in, n_tok)
        dx = torch.from_numpy(x).cuda()
        ys = [torch.full((n_tok, n), float("nan"), dtype=torch.float32, device="cuda") for _, n in proj]
        chart.gemm_group_f32_dev(dev, W, dx.data_ptr(), n_tok, [y.data_ptr() for y in ys], stream())
        assert dev.sync_status(stream()) == 0
        for (t, n), raw, y in zip(proj, raws, ys):
            Y = y.cpu().numpy()
            for c in (0, 77, 159):
                oracle_rows(t, raw, n_in, np.arange(n), x[c], Y[c], f"group part t{t} n{n} col {c}")
        for w in W:
            w.free()
    finally:
        dev.set_gemm_design(Q8_0, chart.Device.GEMM_AUTO)
