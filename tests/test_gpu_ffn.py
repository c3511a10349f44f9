"""GPU parity of the fused FFN in launch form (ah_ffn_gate_up_dev / ah_ffn_dev, through the C ABI).

The reference's fused FFN (ffn_q8act_prepared_into, chart/ffn.rs:1609; fused_ffn_task,
chart/ffn.rs:1532-1594) computes gate and up, the SwiGLU h = round_shift_32(silu_fixed(gate) * up)
exactly (ops/ffn.rs:80, ops/silu.rs:18-60, chart/ffn.rs:246-252), requantizes h (quant_act) and
projects it with down.  Here gate/up and the SwiGLU + requantize run in one launch and down in a
second.  Checked against the oracle:
* gate and up (the f32 values the SwiGLU consumed) within 1e-4 * sum|w * xhat| of the contract;
* the hidden QuantAct bit-exact to the oracle's to_q32 -> swiglu -> quant_act of those values;
* down within tolerance of the contract on that QuantAct, and bit-equal to a separate GEMV on it;
* refusals in the reference FFN's order (chart/ffn.rs:1712-1720): input conversion, projection
  outputs, SwiGLU, and the down projection's only when nothing before it refused.
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


def dbuf(n, dtype=torch.float32):
    return torch.full((n,), float("nan") if dtype == torch.float32 else 0, dtype=dtype, device="cuda")


def check(t, raw, n_in, x, y, rows=None, what=""):
    rb = synth.row_bytes(t, n_in)
    if rows is None:
        rows = np.arange(len(y))
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
    if isinstance(x, tuple):
        codes, scales = x
    else:
        st, codes, scales = oracle.quant_act_f32(x)
        assert st == 0
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


@pytest.mark.parametrize("gu_type,down_type,n_embd,n_ff", [
    (Q4_K, Q6_K, 1536, 8960),   # configs[4] FFN (Q6_K down layers)
    (Q4_K, Q4_K, 1536, 8960),   # configs[4] FFN (Q4_K down layers)
    (Q4_K, Q4_K, 896, 4864),    # configs[1] FFN
    (Q8_0, Q8_0, 256, 300),     # ragged hidden width (a partial last block)
    (Q6_K, Q5_0, 512, 1000),
    (Q5_0, Q8_0, 96, 4000),     # several hidden blocks per workgroup
    (Q3_K, Q2_K, 512, 1000),    # the K-quant families with no GEMM form of their own
    (Q2_K, Q3_K, 256, 300),
])
def test_ffn_vs_oracle(dev, gu_type, down_type, n_embd, n_ff):
    rng = synth.rng_for(11, n_ff + gu_type)
    raws = [scaled_payload(gu_type, rng, n_ff, n_embd, 1 / 32), scaled_payload(gu_type, rng, n_ff, n_embd, 1 / 32),
            scaled_payload(down_type, rng, n_embd, n_ff, 1 / 32)]
    G = dev.upload(gu_type, raws[0], n_ff, n_embd)
    U = dev.upload(gu_type, raws[1], n_ff, n_embd)
    D = dev.upload(down_type, raws[2], n_embd, n_ff)
    x = torch.from_numpy(synth.activations(rng, n_embd)).cuda()
    g, u, y = dbuf(n_ff), dbuf(n_ff), dbuf(n_embd)
    hc = torch.zeros(n_ff + 4, dtype=torch.int8, device="cuda")
    hs = torch.zeros(-(-n_ff // 32), dtype=torch.int64, device="cuda")
    chart.ffn_gate_up_dev(dev, G, U, x.data_ptr(), hc.data_ptr(), hs.data_ptr(), g.data_ptr(), u.data_ptr(), stream())
    assert dev.sync_status(stream()) == 0
    xs, GY, UY = x.cpu().numpy(), g.cpu().numpy(), u.cpu().numpy()
    rows = np.unique(np.concatenate([rng.integers(0, n_ff, 160), [0, n_ff - 1]]))
    check(gu_type, raws[0], n_embd, xs, GY, rows, "gate")
    check(gu_type, raws[1], n_embd, xs, UY, rows, "up")
    st, codes, scales, _ = oracle.swiglu_quant_f32(GY, UY)
    assert st == 0
    assert (hc.cpu().numpy()[:n_ff] == codes).all() and (hs.cpu().numpy() == scales).all()
    # the whole FFN: the same hidden QuantAct, then down within tolerance and equal to a separate GEMV
    hc2 = torch.zeros_like(hc)
    hs2 = torch.zeros_like(hs)
    chart.ffn_dev(dev, G, U, D, x.data_ptr(), y.data_ptr(), hc2.data_ptr(), hs2.data_ptr(), stream())
    assert dev.sync_status(stream()) == 0
    assert torch.equal(hc2[:n_ff], hc[:n_ff]) and torch.equal(hs2, hs)
    check(down_type, raws[2], n_ff, (codes, scales), y.cpu().numpy(), what="down")
    y2 = dbuf(n_embd)
    D.gemv_q8_dev(hc.data_ptr(), hs.data_ptr(), y2.data_ptr(), stream())
    assert dev.sync_status(stream()) == 0
    assert torch.equal(y, y2)
    # from the input's QuantAct (ffn_q8act_prepared_into's `quantize(x)`): the same activation in
    # the workgroups' LDS, so the same hidden QuantAct and output bit for bit
    st, qc, qs = oracle.quant_act_f32(xs)
    assert st == 0
    dqc = torch.zeros(n_embd + 4, dtype=torch.int8, device="cuda")
    dqc[:n_embd] = torch.from_numpy(qc).cuda()
    dqs = torch.from_numpy(qs).cuda()
    y3 = dbuf(n_embd)
    hc3, hs3 = torch.zeros_like(hc), torch.zeros_like(hs)
    chart.ffn_q8_dev(dev, G, U, D, dqc.data_ptr(), dqs.data_ptr(), y3.data_ptr(), hc3.data_ptr(), hs3.data_ptr(),
                     stream())
    assert dev.sync_status(stream()) == 0
    assert torch.equal(hc3[:n_ff], hc[:n_ff]) and torch.equal(hs3, hs) and torch.equal(y3, y)
    for w in (G, U, D):
        w.free()


def big_row_payload(rng, n_out, n_in, hot_rows, d_hot):
    """Q8_0 rows with d = 2^-8 except `hot_rows`, whose blocks carry d_hot and codes 127."""
    raw = synth.payload(Q8_0, rng, n_out, n_in).copy()
    blk = raw.reshape(n_out, -1, 34)
    blk[:, :, 0:2] = np.array([0x1C00], np.uint16).view(np.uint8)  # f16 2^-8
    for r in hot_rows:
        blk[r, :, 0:2] = np.array([d_hot], np.uint16).view(np.uint8)
        blk[r, :, 2:] = 127
    return raw


def test_ffn_refusal_order(dev):
    """SwiGLU overflow at a hidden element refuses with AH_ERR_FFN_OVERFLOW (12) even when the down
    projection also overflows; a non-finite input refuses first (10); the down projection's own
    refusal (OutputOverflow, 9) is reported when the FFN's hidden activation is fine."""
    rng = synth.rng_for(11, 5)
    n_embd, n_ff = 64, 256
    x_np = np.full(n_embd, 4.0, np.float32)
    # gate/up row 40: d = 2^12, codes 127 -> 64 * 127 * 4 * 2^12 ~ 2^27.0 each: silu(g) * u leaves i64
    G = dev.upload(Q8_0, big_row_payload(rng, n_ff, n_embd, [40], 0x6C00), n_ff, n_embd)
    U = dev.upload(Q8_0, big_row_payload(rng, n_ff, n_embd, [40], 0x6C00), n_ff, n_embd)
    G0 = dev.upload(Q8_0, big_row_payload(rng, n_ff, n_embd, [], 0x1C00), n_ff, n_embd)
    U0 = dev.upload(Q8_0, big_row_payload(rng, n_ff, n_embd, [], 0x1C00), n_ff, n_embd)
    # down row 3 with the largest scale: |y| >= 2^31 on any nonzero hidden vector of this size
    dbig_raw = big_row_payload(rng, n_embd, n_ff, [3], 0x7BFF)
    Dbig = dev.upload(Q8_0, dbig_raw, n_embd, n_ff)
    x = torch.from_numpy(x_np).cuda()
    y = dbuf(n_embd)
    hc = torch.zeros(n_ff, dtype=torch.int8, device="cuda")
    hs = torch.zeros(n_ff // 32, dtype=torch.int64, device="cuda")
    g, u = dbuf(n_ff), dbuf(n_ff)
    chart.ffn_gate_up_dev(dev, G, U, x.data_ptr(), hc.data_ptr(), hs.data_ptr(), g.data_ptr(), u.data_ptr(), stream())
    torch.cuda.synchronize()
    # the oracle refuses the same gate / up values at the same step
    assert oracle.swiglu_quant_f32(g.cpu().numpy(), u.cpu().numpy())[0] == 12
    assert dev.sync_status(stream()) == 12
    # the down projection overflows too, but the hidden activation's refusal comes first
    chart.ffn_dev(dev, G, U, Dbig, x.data_ptr(), y.data_ptr(), hc.data_ptr(), hs.data_ptr(), stream())
    assert dev.sync_status(stream()) == 12
    # a fine hidden activation: the down projection's own refusal is reported
    chart.ffn_dev(dev, G0, U0, Dbig, x.data_ptr(), y.data_ptr(), hc.data_ptr(), hs.data_ptr(), stream())
    assert dev.sync_status(stream()) == 9
    # (the contract refuses that hidden activation's down projection the same way)
    assert oracle.matvec_q8act(Q8_0, dbig_raw, n_embd, n_ff, hc.cpu().numpy(), hs.cpu().numpy())[0] == 9
    # the input's conversion refuses before everything else
    xb = x.clone()
    xb[7] = float("inf")
    chart.ffn_dev(dev, G, U, Dbig, xb.data_ptr(), y.data_ptr(), hc.data_ptr(), hs.data_ptr(), stream())
    assert dev.sync_status(stream()) == 10
    # and the status is clear again afterwards
    D = dev.upload(Q8_0, synth.payload(Q8_0, rng, n_embd, n_ff), n_embd, n_ff)
    chart.ffn_dev(dev, G0, U0, D, x.data_ptr(), y.data_ptr(), hc.data_ptr(), hs.data_ptr(), stream())
    assert dev.sync_status(stream()) == 0
    for w in (G, U, G0, U0, Dbig, D):
        w.free()


def test_ffn_argument_refusals(dev):
    rng = synth.rng_for(11, 6)
    G = dev.upload(Q4_K, synth.payload(Q4_K, rng, 256, 512), 256, 512)
    U = dev.upload(Q4_K, synth.payload(Q4_K, rng, 256, 512), 256, 512)
    U2 = dev.upload(Q4_K, synth.payload(Q4_K, rng, 128, 512), 128, 512)
    D = dev.upload(Q8_0, synth.payload(Q8_0, rng, 512, 256), 512, 256)
    x = torch.zeros(512, device="cuda")
    hc = torch.zeros(256, dtype=torch.int8, device="cuda")
    hs = torch.zeros(8, dtype=torch.int64, device="cuda")
    y = torch.zeros(512, device="cuda")
    with pytest.raises(chart.MatvecError):  # gate and up of different shapes
        chart.ffn_gate_up_dev(dev, G, U2, x.data_ptr(), hc.data_ptr(), hs.data_ptr())
    with pytest.raises(chart.MatvecError):  # down does not map n_ff back to n_embd
        chart.ffn_dev(dev, G, U, U, x.data_ptr(), y.data_ptr(), hc.data_ptr(), hs.data_ptr())
    chart.ffn_dev(dev, G, U, D, x.data_ptr(), y.data_ptr(), hc.data_ptr(), hs.data_ptr(), stream())
    assert dev.sync_status(stream()) == 0
    assert not y.any()  # a zero input gives a zero hidden vector and a zero output
    for w in (G, U, U2, D):
        w.free()
