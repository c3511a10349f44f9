"""GPU parity of the persistent decode sequence (ah_seq_*): stages in one launch behind grid barriers.

* A chain whose stages read the previous stage's output equals the same projections launched one
  by one (bit for bit), over several runs of one sequence (the barrier state carries over).
* The fused FFN (gate/up -> SwiGLU -> down, chart/ffn.rs:1532-1594): gate/up within tolerance of
  the oracle; the hidden QuantAct bit-exact to the oracle's to_q32 -> silu_fixed -> round_shift_32
  -> quant_act of the GPU's own gate/up (ops/silu.rs:18-60, chart/ffn.rs:246-252); down within
  tolerance of the oracle on that QuantAct and bit-equal to a separate GEMV on it.
* SwiGLU edge values (saturation bounds, +-ln 2, 0, overflow) and refusals reported at their stage.
* A configs[4]-structured token (q/k/v -> o -> gate/up -> SwiGLU -> down per layer, then the Q6_K
  head) against the oracle, stage by stage.
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
ONE = 1 << 32


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
    n_out = len(y) if rows is None else None
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


def small_payload(t, rng, n_out, n_in, scale):
    """A synthetic payload whose block scales are multiplied by `scale` (keeps chained outputs
    of moderate size)."""
    raw = synth.payload(t, rng, n_out, n_in).copy()
    qk, bb = synth.GEOM[t]
    blk = raw.reshape(-1, bb)
    for off in (o for o in synth.SCALE_AT[t] if o is not None):
        d = blk[:, off:off + 2].copy().view(np.float16).astype(np.float32) * scale
        blk[:, off:off + 2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return raw


def test_seq_chain_equals_separate_launches(dev):
    rng = synth.rng_for(9, 1)
    shapes = [(Q4_K, 896, 896), (Q6_K, 1536, 896), (Q8_0, 640, 1536), (Q4_K, 256, 640)]
    W, raws = [], []
    for t, n_out, n_in in shapes:
        raw = small_payload(t, rng, n_out, n_in, 1.0 / 16)
        raws.append(raw)
        W.append(dev.upload(t, raw, n_out, n_in))
    x0 = torch.from_numpy(synth.activations(rng, 896)).cuda()
    ys = [dbuf(n_out) for _, n_out, _ in shapes]
    # stage 0: parts 0 (x0) ; stage 1: part 1 reads y0 ; stage 2: part 2 reads y1 ; stage 3: part 3 reads y2
    seq = chart.Seq(dev, [("gemv", [(W[0], x0.data_ptr(), ys[0].data_ptr())]),
                          ("gemv", [(W[1], ys[0].data_ptr(), ys[1].data_ptr())]),
                          ("gemv", [(W[2], ys[1].data_ptr(), ys[2].data_ptr())]),
                          ("gemv", [(W[3], ys[2].data_ptr(), ys[3].data_ptr())])])
    ref = [dbuf(n_out) for _, n_out, _ in shapes]
    inp = x0
    for w, y in zip(W, ref):
        w.gemv_f32_dev(inp.data_ptr(), y.data_ptr(), stream())
        inp = y
    assert dev.sync_status(stream()) == 0
    for run in range(4):
        for y in ys:
            y.fill_(float("nan"))
        seq.run(stream())
        assert seq.sync_status(stream()) == (0, 0)
        for i, (y, r) in enumerate(zip(ys, ref)):
            assert torch.equal(y, r), (run, i)
    # and each stage against the oracle on its own input
    inputs = [x0] + ys[:-1]
    for (t, n_out, n_in), raw, x, y in zip(shapes, raws, inputs, ys):
        check(t, raw, n_in, x.cpu().numpy(), y.cpu().numpy(), what=f"chain t{t}")
    seq.free()
    for w in W:
        w.free()


def ffn_case(dev, rng, n_embd, n_ff, down_type, sigma=1.0 / 32):
    raws = [small_payload(Q4_K, rng, n_ff, n_embd, sigma), small_payload(Q4_K, rng, n_ff, n_embd, sigma),
            small_payload(down_type, rng, n_embd, n_ff, sigma)]
    W = [dev.upload(Q4_K, raws[0], n_ff, n_embd), dev.upload(Q4_K, raws[1], n_ff, n_embd),
         dev.upload(down_type, raws[2], n_embd, n_ff)]
    return raws, W


@pytest.mark.parametrize("n_embd,n_ff,down_type", [(1536, 8960, Q6_K), (896, 4864, Q4_K), (256, 300, Q8_0),
                                                    (896, 4864, Q5_0), (512, 1000, Q3_K)])
def test_seq_fused_ffn_vs_oracle(dev, n_embd, n_ff, down_type):
    rng = synth.rng_for(9, n_ff)
    raws, W = ffn_case(dev, rng, n_embd, n_ff, down_type)
    x = torch.from_numpy(synth.activations(rng, n_embd)).cuda()
    g, u, y = dbuf(n_ff), dbuf(n_ff), dbuf(n_embd)
    hc = torch.zeros(n_ff + 8, dtype=torch.int8, device="cuda")
    hs = torch.zeros(-(-n_ff // 32), dtype=torch.int64, device="cuda")
    seq = chart.Seq(dev, [("gemv", [(W[0], x.data_ptr(), g.data_ptr()), (W[1], x.data_ptr(), u.data_ptr())]),
                          ("swiglu", g.data_ptr(), u.data_ptr(), n_ff, hc.data_ptr(), hs.data_ptr()),
                          ("gemv", [(W[2], (hc.data_ptr(), hs.data_ptr()), y.data_ptr())])])
    seq.run(stream())
    assert seq.sync_status(stream()) == (0, 0)
    xs = x.cpu().numpy()
    G, U, Y = g.cpu().numpy(), u.cpu().numpy(), y.cpu().numpy()
    rows = np.unique(rng.integers(0, n_ff, 128))
    check(Q4_K, raws[0], n_embd, xs, G, rows, "gate")
    check(Q4_K, raws[1], n_embd, xs, U, rows, "up")
    st, codes, scales, _ = oracle.swiglu_quant_f32(G, U)
    assert st == 0
    HC, HS = hc.cpu().numpy()[:n_ff], hs.cpu().numpy()
    assert (HC == codes).all() and (HS == scales).all()
    check(down_type, raws[2], n_ff, (codes, scales), Y, what="down")
    # the down stage equals a separate GEMV on the same QuantAct
    y2 = dbuf(n_embd)
    W[2].gemv_q8_dev(hc.data_ptr(), hs.data_ptr(), y2.data_ptr(), stream())
    assert dev.sync_status(stream()) == 0
    assert torch.equal(y, y2)
    seq.free()
    for w in W:
        w.free()


def test_seq_swiglu_edge_values_and_refusals(dev):
    n = 96
    vals = [0.0, 2977044472 / ONE, -2977044472 / ONE, 16.0, -21.0, 16.5, -21.5, 1e-9, -1e-9, 3.0, -3.0,
            15.999, -20.999, 100.0, -100.0, 0.5]
    gate = np.resize(np.array(vals, np.float32), n)
    up = np.random.default_rng(3).standard_normal(n).astype(np.float32)
    dg, du = torch.from_numpy(gate).cuda(), torch.from_numpy(up).cuda()
    hc = torch.zeros(n, dtype=torch.int8, device="cuda")
    hs = torch.zeros(n // 32, dtype=torch.int64, device="cuda")
    seq = chart.Seq(dev, [("swiglu", dg.data_ptr(), du.data_ptr(), n, hc.data_ptr(), hs.data_ptr())])
    seq.run(stream())
    assert seq.sync_status(stream()) == (0, 0)
    st, codes, scales, _ = oracle.swiglu_quant_f32(gate, up)
    assert st == 0 and (hc.cpu().numpy() == codes).all() and (hs.cpu().numpy() == scales).all()
    # overflow: silu(2^30) * 2^30 leaves i64 -> FfnError::Overflow at that element
    gate2, up2 = gate.copy(), up.copy()
    gate2[40], up2[40] = 2.0 ** 30, 2.0 ** 30
    assert oracle.swiglu_quant_f32(gate2, up2)[0] == 12
    dg.copy_(torch.from_numpy(gate2))
    du.copy_(torch.from_numpy(up2))
    seq.run(stream())
    assert seq.sync_status(stream()) == (12, 0)
    # a non-finite gate is the conversion's refusal
    gate2[40], gate2[41] = 1.0, float("inf")
    dg.copy_(torch.from_numpy(gate2))
    seq.run(stream())
    assert seq.sync_status(stream()) == (10, 0)
    seq.free()


def test_seq_refusal_reported_at_its_stage(dev):
    rng = synth.rng_for(9, 7)
    raw = small_payload(Q4_K, rng, 256, 512, 1.0)
    w = dev.upload(Q4_K, raw, 256, 512)
    x = torch.from_numpy(synth.activations(rng, 512)).cuda()
    xb = x.clone()
    xb[100] = float("inf")
    y0, y1 = dbuf(256), dbuf(256)
    seq = chart.Seq(dev, [("gemv", [(w, x.data_ptr(), y0.data_ptr())]), ("gemv", [(w, xb.data_ptr(), y1.data_ptr())])])
    seq.run(stream())
    assert seq.sync_status(stream()) == (10, 1)
    seq.run(stream())
    assert seq.sync_status(stream()) == (10, 1)
    xb[100] = 1.0
    seq.run(stream())
    assert seq.sync_status(stream()) == (0, 0)
    seq.free()
    w.free()


def test_seq_config4_token_vs_oracle(dev):
    """Two configs[4] layers (the second with its Q4_K ffn_down) and the Q6_K vocab head, as one
    token: q/k/v -> o -> gate/up -> SwiGLU -> down per layer, then the head.  Inputs of q/k/v, o
    and the head are their own buffers (the engine's attention, norms and residuals run between
    them and are not on this path); down reads the SwiGLU stage's QuantAct."""
    rng = synth.rng_for(9, 44)
    stages, checks, keep = [], [], []
    for l, down_t in ((0, Q6_K), (3, Q4_K)):
        spec = [("q", Q4_K, 1536, 1536), ("k", Q4_K, 256, 1536), ("v", Q6_K, 256, 1536), ("o", Q4_K, 1536, 1536),
                ("gate", Q4_K, 8960, 1536), ("up", Q4_K, 8960, 1536), ("down", down_t, 1536, 8960)]
        L = {}
        for name, t, n_out, n_in in spec:
            raw = small_payload(t, rng, n_out, n_in, 1.0 / 32)
            L[name] = (t, n_out, n_in, raw, dev.upload(t, raw, n_out, n_in), dbuf(n_out))
        xa = torch.from_numpy(synth.activations(rng, 1536)).cuda()
        xo = torch.from_numpy(synth.activations(rng, 1536)).cuda()
        xf = torch.from_numpy(synth.activations(rng, 1536)).cuda()
        hc = torch.zeros(8960, dtype=torch.int8, device="cuda")
        hs = torch.zeros(280, dtype=torch.int64, device="cuda")
        keep += [L, xa, xo, xf, hc, hs]
        part = lambda nm, x: (L[nm][4], x, L[nm][5].data_ptr())
        stages += [("gemv", [part("q", xa.data_ptr()), part("k", xa.data_ptr()), part("v", xa.data_ptr())]),
                   ("gemv", [part("o", xo.data_ptr())]),
                   ("gemv", [part("gate", xf.data_ptr()), part("up", xf.data_ptr())]),
                   ("swiglu", L["gate"][5].data_ptr(), L["up"][5].data_ptr(), 8960, hc.data_ptr(), hs.data_ptr()),
                   ("gemv", [part("down", (hc.data_ptr(), hs.data_ptr()))])]
        checks.append((L, xa, xo, xf, hc, hs))
    raw_h = synth.payload(Q6_K, rng, 151936, 1536)
    wh = dev.upload(Q6_K, raw_h, 151936, 1536)
    xh, yh = torch.from_numpy(synth.activations(rng, 1536)).cuda(), dbuf(151936)
    stages.append(("gemv", [(wh, xh.data_ptr(), yh.data_ptr())]))
    seq = chart.Seq(dev, stages)
    for _ in range(2):
        seq.run(stream())
        assert seq.sync_status(stream()) == (0, 0)
    for L, xa, xo, xf, hc, hs in checks:
        ins = {"q": xa, "k": xa, "v": xa, "o": xo, "gate": xf, "up": xf}
        for name, (t, n_out, n_in, raw, w, y) in L.items():
            rows = np.unique(np.concatenate([np.arange(4), rng.integers(0, n_out, 48), [n_out - 1]]))
            if name == "down":
                x = (hc.cpu().numpy(), hs.cpu().numpy())
            else:
                x = ins[name].cpu().numpy()
            check(t, raw, n_in, x, y.cpu().numpy(), rows, f"layer {name}")
        st, codes, scales, _ = oracle.swiglu_quant_f32(L["gate"][5].cpu().numpy(), L["up"][5].cpu().numpy())
        assert st == 0 and (hc.cpu().numpy() == codes).all() and (hs.cpu().numpy() == scales).all()
    rows = np.unique(np.concatenate([np.arange(8), rng.integers(0, 151936, 64), [151935]]))
    check(Q6_K, raw_h, 1536, xh.cpu().numpy(), yh.cpu().numpy(), rows, "head")
    seq.free()
    wh.free()
    for L, *_ in checks:
        for v in L.values():
            v[4].free()


def test_seq_timeout_then_whole_run(dev):
    """A grid-barrier wait that gives up (a one-poll limit set from the host) reports
    AH_ERR_SEQ_TIMEOUT at a waiting stage and every workgroup still finishes the launch; the next
    runs with the default limit are whole runs again, equal to separate launches bit for bit."""
    rng = synth.rng_for(9, 7)
    shapes = [(Q4_K, 8960, 1536), (Q6_K, 1536, 8960), (Q8_0, 640, 1536), (Q4_K, 256, 640)]
    W = [dev.upload(t, small_payload(t, rng, n_out, n_in, 1.0 / 16), n_out, n_in) for t, n_out, n_in in shapes]
    x0 = torch.from_numpy(synth.activations(rng, 1536)).cuda()
    ys = [dbuf(n_out) for _, n_out, _ in shapes]
    inputs = [x0] + ys[:-1]
    seq = chart.Seq(dev, [("gemv", [(w, x.data_ptr(), y.data_ptr())]) for w, x, y in zip(W, inputs, ys)])
    ref = [dbuf(n_out) for _, n_out, _ in shapes]
    inp = x0
    for w, y in zip(W, ref):
        w.gemv_f32_dev(inp.data_ptr(), y.data_ptr(), stream())
        inp = y
    assert dev.sync_status(stream()) == 0
    seq.set_spin_limit(1)
    seq.run(stream())
    st, stage = seq.sync_status(stream())
    assert st == 25 and 1 <= stage < len(shapes), (st, stage)
    seq.set_spin_limit(0)
    for run in range(2):
        for y in ys:
            y.fill_(float("nan"))
        seq.run(stream())
        assert seq.sync_status(stream()) == (0, 0)
        for i, (y, r) in enumerate(zip(ys, ref)):
            assert torch.equal(y, r), (run, i)
    seq.free()
    for w in W:
        w.free()
