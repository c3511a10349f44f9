"""GPU parity of the prefill FFN (ah_ffn_gate_up_prefill_dev / ah_ffn_prefill_dev, N > 1).

The reference's column path (step/cols.rs:1026-1067) quantizes the N input columns, runs the
[W_gate; W_up] GEMM with the SwiGLU epilogue (gemm_q8_0_swiglu_carrier, kern/gemm.rs:955-1168)
or the gate and up projections then swiglu_cols (chart/ffn.rs:493-560), and projects the hidden
columns with down (their quant_act first).  Here Q4_K / Q2_K / Q3_K gate/up run as one launch of
the dequantize-once tiles with the SwiGLU + hidden quantizer in the epilogue; other types as the
grouped GEMM plus a SwiGLU pass.  Checked against the oracle:
* gate and up (the f32 values the SwiGLU consumed) within 1e-4 * sum|w * xhat| of the contract;
* every token's hidden QuantAct bit-exact to the oracle's to_q32 -> swiglu -> quant_act of those
  values (the F32 carrier);
* down within tolerance of the contract on that QuantAct, and bit-equal to a separate GEMM on it;
* refusals in the reference FFN's order: the input's quantization, the gate projection (all
  tokens), the up projection, the SwiGLU elements, and the down projection only when nothing
  before it refused.
"""
import numpy as np
import pytest

import oracle
from apeiron_amd import chart, synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-4
Q32 = 2.0 ** -32
Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q6_K = 6, 8, 10, 11, 12, 14


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    d = chart.Device(0)
    yield d
    d.close()


def stream():
    return torch.cuda.current_stream().cuda_stream


def nan2d(n, m):
    return torch.full((n, m), float("nan"), dtype=torch.float32, device="cuda")


def check_rows(t, raw, n_in, codes, scales, y, rows, what):
    rb = synth.row_bytes(t, n_in)
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
    st, yref = oracle.matvec_q8act(t, sub, len(rows), n_in, codes, scales)
    st2, absdot = oracle.row_absdot(t, sub, len(rows), n_in, codes, scales)
    assert st == 0 and st2 == 0, (what, st, st2)
    err = np.abs(np.asarray(y, np.float64)[rows] - yref.astype(np.float64) * Q32)
    bad = np.nonzero(err > TOL * absdot + Q32)[0]
    assert bad.size == 0, f"{what}: rows {rows[bad[:6]]} err {err[bad[:6]]} tol {(TOL * absdot)[bad[:6]]}"


def scaled_payload(t, rng, n_out, n_in, scale):
    """A synthetic payload whose block scales are multiplied by `scale` (moderate hidden values)."""
    raw = synth.payload(t, rng, n_out, n_in).copy()
    qk, bb = synth.GEOM[t]
    blk = raw.reshape(-1, bb)
    for off in (o for o in synth.SCALE_AT[t] if o is not None):
        d = blk[:, off:off + 2].copy().view(np.float16).astype(np.float32) * scale
        blk[:, off:off + 2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return raw


def run_case(dev, gu_type, down_type, n_embd, n_ff, n_tok, fused, spread=False, seed=0):
    rng = synth.rng_for(12, n_ff + gu_type + 7 * n_tok + seed)
    raws = [scaled_payload(gu_type, rng, n_ff, n_embd, 1 / 32), scaled_payload(gu_type, rng, n_ff, n_embd, 1 / 32),
            scaled_payload(down_type, rng, n_embd, n_ff, 1 / 32)]
    G = dev.upload(gu_type, raws[0], n_ff, n_embd)
    U = dev.upload(gu_type, raws[1], n_ff, n_embd)
    D = dev.upload(down_type, raws[2], n_embd, n_ff)
    xn = synth.activations(rng, n_embd, n_tok).reshape(n_tok, n_embd).astype(np.float32)
    if spread:  # every third token's blocks span ~40 binades (2^-36 .. 2^4, the largest small
        # enough that the SwiGLU stays in range): the tiles' exact path serves them
        nb = n_embd // 32
        for tok in range(0, n_tok, 3):
            xn[tok] *= np.repeat(np.exp2(np.arange(nb) * 40.0 / nb - 36.0), 32).astype(np.float32)
    x = torch.from_numpy(xn).cuda()
    nbh = -(-n_ff // 32)
    gy, uy = nan2d(n_tok, n_ff), nan2d(n_tok, n_ff)
    hc = torch.zeros((n_tok, n_ff), dtype=torch.int8, device="cuda")
    hs = torch.zeros((n_tok, nbh), dtype=torch.int64, device="cuda")
    dev.set_ffn_prefill_form(chart.Device.FFN_FUSED if fused else chart.Device.FFN_TWO_PASS)
    try:
        chart.ffn_gate_up_prefill_dev(dev, G, U, x.data_ptr(), n_tok, hc.data_ptr(), hs.data_ptr(),
                                      gy.data_ptr(), uy.data_ptr(), stream())
        assert dev.sync_status(stream()) == 0
        GY, UY, HC, HS = gy.cpu().numpy(), uy.cpu().numpy(), hc.cpu().numpy(), hs.cpu().numpy()
        # every token's hidden QuantAct, bit for bit
        for t in range(n_tok):
            st, codes, scales, _ = oracle.swiglu_quant_f32(GY[t], UY[t])
            assert st == 0, t
            assert (HC[t] == codes).all() and (HS[t] == scales).all(), f"token {t}"
        # gate and up on sampled tokens and rows
        rows = np.unique(np.concatenate([rng.integers(0, n_ff, 96), [0, n_ff - 1]]))
        toks = sorted({0, n_tok - 1, n_tok // 2, min(n_tok - 1, 63), min(n_tok - 1, 64), min(n_tok - 1, 129)})
        for t in toks:
            st, codes, scales = oracle.quant_act_f32(xn[t])
            assert st == 0
            check_rows(gu_type, raws[0], n_embd, codes, scales, GY[t], rows, f"gate token {t}")
            check_rows(gu_type, raws[1], n_embd, codes, scales, UY[t], rows, f"up token {t}")
        # the whole FFN: the same hidden QuantAct, down within tolerance and equal to a GEMM on it
        y = nan2d(n_tok, n_embd)
        hc2, hs2 = torch.zeros_like(hc), torch.zeros_like(hs)
        chart.ffn_prefill_dev(dev, G, U, D, x.data_ptr(), n_tok, y.data_ptr(), hc2.data_ptr(), hs2.data_ptr(),
                              stream())
        assert dev.sync_status(stream()) == 0
        assert torch.equal(hc2, hc) and torch.equal(hs2, hs)
        Y = y.cpu().numpy()
        drows = np.unique(np.concatenate([rng.integers(0, n_embd, 64), [0, n_embd - 1]]))
        for t in toks:
            check_rows(down_type, raws[2], n_ff, HC[t], HS[t], Y[t], drows, f"down token {t}")
        y2 = nan2d(n_tok, n_embd)
        D.gemm_q8_dev(hc.data_ptr(), hs.data_ptr(), n_tok, y2.data_ptr(), stream())
        assert dev.sync_status(stream()) == 0
        assert torch.equal(y, y2)
        # from the tokens' QuantActs (the engine's own quantized columns): the same operand, so the
        # same hidden QuantAct and outputs bit for bit
        st, qc, qs = oracle.quant_act_f32_batch(xn)
        assert st == 0
        dqc, dqs = torch.from_numpy(qc).cuda(), torch.from_numpy(qs).cuda()
        y3 = nan2d(n_tok, n_embd)
        hc3, hs3 = torch.zeros_like(hc), torch.zeros_like(hs)
        chart.ffn_prefill_q8_dev(dev, G, U, D, dqc.data_ptr(), dqs.data_ptr(), n_tok, y3.data_ptr(), hc3.data_ptr(),
                                 hs3.data_ptr(), stream())
        assert dev.sync_status(stream()) == 0
        assert torch.equal(hc3, hc) and torch.equal(hs3, hs) and torch.equal(y3, y)
    finally:
        dev.set_ffn_prefill_form(chart.Device.FFN_AUTO)
        for w in (G, U, D):
            w.free()


@pytest.mark.parametrize("gu_type,down_type,n_embd,n_ff,n_tok,fused", [
    (Q4_K, Q6_K, 1536, 8960, 512, True),    # configs[4] FFN (Q6_K down layers), one launch
    (Q4_K, Q4_K, 1536, 8960, 512, False),   # the same shape, two passes
    (Q4_K, Q4_K, 896, 4864, 77, True),      # configs[1] FFN, a partial token tile
    (Q2_K, Q3_K, 512, 1000, 33, True),      # hidden width past whole tiles and a partial block
    (Q2_K, Q3_K, 512, 1000, 33, False),
    (Q3_K, Q2_K, 256, 300, 130, True),
    (Q8_0, Q8_0, 256, 300, 40, True),       # types without the tile form: two passes
    (Q6_K, Q5_0, 512, 1000, 20, True),
    (Q5_0, Q8_0, 96, 200, 9, True),
])
def test_ffn_prefill_vs_oracle(dev, gu_type, down_type, n_embd, n_ff, n_tok, fused):
    run_case(dev, gu_type, down_type, n_embd, n_ff, n_tok, fused)


@pytest.mark.parametrize("gu_type,down_type,n_embd,n_ff,n_tok", [
    (Q4_K, Q4_K, 896, 4864, 77),   # configs[1] FFN shapes, gate/up and down on the int8 design
    (Q4_K, Q8_0, 512, 1000, 33),   # a Q8_0 down on its int8 design, a partial block
])
def test_ffn_prefill_two_pass_int8_designs(dev, gu_type, down_type, n_embd, n_ff, n_tok):
    """The two-pass FFN with the int8 GEMM designs selected (ah_set_gemm_design): the hidden
    QuantAct bit for bit, gate/up and down within tolerance, down equal to a GEMM on the codes."""
    for t in {gu_type, down_type}:
        dev.set_gemm_design(t, chart.Device.GEMM_INT8)
    try:
        run_case(dev, gu_type, down_type, n_embd, n_ff, n_tok, False)
    finally:
        for t in {gu_type, down_type}:
            dev.set_gemm_design(t, chart.Device.GEMM_AUTO)


@pytest.mark.parametrize("gu_type", [Q4_K, Q3_K])
def test_ffn_prefill_wide_spread_tokens(dev, gu_type):
    """Tokens no f16 band can carry: the fused epilogue takes their gate / up from the exact path."""
    run_case(dev, gu_type, Q8_0, 1536, 320, 40, True, spread=True)


def const_payload(t, n_out, n_in, d_bits):
    """Every weight equal to the f16 `d_bits`: Q4_K with sc = 1, m = 0, codes 1 and dmin 0; Q8_0
    with codes 1."""
    if t == Q8_0:
        blk = np.zeros((n_out * n_in // 32, 34), np.uint8)
        blk[:, 0], blk[:, 1] = d_bits & 0xFF, d_bits >> 8
        blk[:, 2:] = 1
        return blk.reshape(-1)
    n = n_out * n_in // 256
    blk = np.zeros((n, 144), np.uint8)
    blk[:, 0], blk[:, 1] = d_bits & 0xFF, d_bits >> 8
    blk[:, 4:16] = synth.pack_q4_k_scales(np.ones((n, 8), np.uint8), np.zeros((n, 8), np.uint8))
    blk[:, 16:] = 0x11
    return blk.reshape(-1)


@pytest.mark.parametrize("t,fused", [(Q4_K, True), (Q4_K, False), (Q8_0, True)])
def test_ffn_prefill_refusal_order(dev, t, fused):
    """Refusals in the order the reference meets them, not token-major: every token's gate output
    before any up output, those before any SwiGLU element, and the down projection last; the
    input's quantization before all of them."""
    n_embd, n_ff = 256, 64
    one, tiny, big = 0x3C00, 0x0C00, 0x7800  # f16 1, 2^-12, 2^15
    G1 = dev.upload(t, const_payload(t, n_ff, n_embd, one), n_ff, n_embd)
    U1 = dev.upload(t, const_payload(t, n_ff, n_embd, one), n_ff, n_embd)
    Gs = dev.upload(t, const_payload(t, n_ff, n_embd, tiny), n_ff, n_embd)
    Dbig = dev.upload(Q8_0, const_payload(Q8_0, n_embd, n_ff, big), n_embd, n_ff)
    hc = torch.zeros((2, n_ff), dtype=torch.int8, device="cuda")
    hs = torch.zeros((2, 2), dtype=torch.int64, device="cuda")
    y = nan2d(2, n_embd)

    def gate_up(G, U, c0, c1):
        x = torch.tensor(np.stack([np.full(n_embd, c0, np.float32), np.full(n_embd, c1, np.float32)])).cuda()
        chart.ffn_gate_up_prefill_dev(dev, G, U, x.data_ptr(), 2, hc.data_ptr(), hs.data_ptr(), None, None, stream())
        return dev.sync_status(stream())

    dev.set_ffn_prefill_form(chart.Device.FFN_FUSED if fused else chart.Device.FFN_TWO_PASS)
    try:
        # token 0: gate = up = 2^16, h = 2^32 leaves i64 (SwiGLU refusal, 12); token 1: gate = up =
        # 2^32 (OutputOverflow, 9).  The gate projection of token 1 comes first.
        assert oracle.swiglu(1 << 48, 1 << 48)[0] == 12
        assert gate_up(G1, U1, 2.0 ** 8, 2.0 ** 24) == 9
        assert gate_up(G1, U1, 2.0 ** 8, 1.0) == 12  # token 0 alone
        # gate = 2^-12 * up: token 0 gate 2^10, up 2^22 (SwiGLU 12); token 1 gate 2^20 (fine), up
        # 2^32 (9): the up projection comes before the SwiGLU of any token
        assert gate_up(Gs, U1, 2.0 ** 14, 2.0 ** 24) == 9
        assert gate_up(Gs, U1, 2.0 ** 14, 1.0) == 12
        # the input's quantization first: token 1 non-finite, token 0 overflowing its gate
        assert gate_up(G1, U1, 2.0 ** 24, float("inf")) == 10
        # the down projection's refusal only when nothing before it refused
        x = torch.tensor(np.stack([np.full(n_embd, 1.0, np.float32), np.full(n_embd, 2.0 ** 8, np.float32)])).cuda()
        chart.ffn_prefill_dev(dev, G1, U1, Dbig, x.data_ptr(), 2, y.data_ptr(), hc.data_ptr(), hs.data_ptr(),
                              stream())
        assert dev.sync_status(stream()) == 12
        x[1] = 1.0
        chart.ffn_prefill_dev(dev, G1, U1, Dbig, x.data_ptr(), 2, y.data_ptr(), hc.data_ptr(), hs.data_ptr(),
                              stream())
        assert dev.sync_status(stream()) == 9
        # and clear afterwards
        assert gate_up(G1, U1, 1.0, 0.5) == 0
    finally:
        dev.set_ffn_prefill_form(chart.Device.FFN_AUTO)
        for w in (G1, U1, Gs, Dbig):
            w.free()


def test_swiglu_quant_dev_vs_oracle(dev):
    """The standalone SwiGLU pass (swiglu_cols + quant_cols) on f32 gate / up columns, including
    elements that refuse: the first refusal token-major."""
    rng = np.random.default_rng(5)
    n_tok, n_ff = 37, 1000
    g = (rng.standard_normal((n_tok, n_ff)) * 8).astype(np.float32)
    u = (rng.standard_normal((n_tok, n_ff)) * 8).astype(np.float32)
    hc = torch.zeros((n_tok, n_ff), dtype=torch.int8, device="cuda")
    hs = torch.zeros((n_tok, 32), dtype=torch.int64, device="cuda")
    dg, du = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    chart.swiglu_quant_dev(dev, dg.data_ptr(), du.data_ptr(), n_tok, n_ff, hc.data_ptr(), hs.data_ptr(), stream())
    assert dev.sync_status(stream()) == 0
    HC, HS = hc.cpu().numpy(), hs.cpu().numpy()
    for t in range(n_tok):
        st, codes, scales, _ = oracle.swiglu_quant_f32(g[t], u[t])
        assert st == 0 and (HC[t] == codes).all() and (HS[t] == scales).all(), t
    # token 3 element 900 overflows the SwiGLU, token 5 element 2 has a non-finite gate: token 3 first
    g[3, 900], u[3, 900] = 2.0 ** 16, 2.0 ** 16
    g[5, 2] = float("nan")
    dg, du = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    chart.swiglu_quant_dev(dev, dg.data_ptr(), du.data_ptr(), n_tok, n_ff, hc.data_ptr(), hs.data_ptr(), stream())
    assert dev.sync_status(stream()) == oracle.swiglu_quant_f32(g[3], u[3])[0] == 12
