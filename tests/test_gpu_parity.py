"""GPU parity: the HIP path (through the C ABI) against the exact CPU oracle.

Bar (from the path's contract):
  * activation codes and scales: bit-exact to quant_act(to_q32(x));
  * per-group integer dots (D_b per 32, Q6_K per 16): bit-exact, read from inside the
    production GEMV kernel;
  * f32 outputs: |y_gpu - y_ref| <= 1e-4 * sum_i |w_i * xhat_i| + 2^-32 per row, where y_ref is
    the oracle's exact Q32.32 result (the 2^-32 term is the reference's own output quantum).
"""
import os

import numpy as np
import pytest

import oracle
from apeiron_amd import chart, synth
from quant_edges import edge_blocks_f32

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
TOL = 1e-4
Q32 = 2.0 ** -32


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


def ptr(t):
    return t.data_ptr()


def gemv_q8(dev, w, codes, scales, dots=False):
    n_out = w.n_out
    dc, ds = to_dev(codes), to_dev(scales)
    y = torch.empty(max(n_out, 1), dtype=torch.float32, device="cuda")
    if dots:
        ng = -(-w.n_in // 16) if w.ggml_type in (10, 11, 14) else -(-w.n_in // 32)
        dd = torch.full((max(n_out, 1), max(ng, 1)), -7, dtype=torch.int32, device="cuda")
        w.gemv_q8_dots_dev(ptr(dc), ptr(ds), ptr(y), ptr(dd), stream())
        assert dev.sync_status(stream()) == 0
        return y.cpu().numpy()[:n_out], dd.cpu().numpy()[:n_out, :ng]
    w.gemv_q8_dev(ptr(dc), ptr(ds), ptr(y), stream())
    assert dev.sync_status(stream()) == 0
    return y.cpu().numpy()[:n_out]


def assert_close(y, yref_q32, absdot, what=""):
    ref = np.asarray(yref_q32, np.float64) * Q32
    err = np.abs(np.asarray(y, np.float64) - ref)
    tol = TOL * np.asarray(absdot) + Q32
    bad = np.nonzero(err > tol)[0]
    assert bad.size == 0, f"{what}: rows {bad[:8]} err {err[bad[:8]]} tol {tol[bad[:8]]}"


def golden_cases():
    z = np.load(GOLDEN, allow_pickle=False)
    for i in range(int(z["count"])):
        p = f"c{i:03d}_"
        t, rows, n_in = (int(v) for v in z[p + "meta"])
        yield dict(kind=str(z[p + "kind"]), t=t, rows=rows, n_in=n_in, raw=z[p + "raw"], x=z[p + "x"],
                   codes=z[p + "codes"], scales=z[p + "scales"], y=z[p + "y"], dots=z[p + "dots"],
                   xf=z[p + "xf"] if p + "xf" in z else None)


# ---- activation quantizer -----------------------------------------------------------------

def quant_f32_gpu(dev, x2d):
    n_tok, n_in = x2d.shape
    dx = to_dev(x2d.astype(np.float32))
    dc = torch.zeros((n_tok, n_in), dtype=torch.int8, device="cuda")
    ds = torch.zeros((n_tok, -(-n_in // 32)), dtype=torch.int64, device="cuda")
    dev.quant_act_f32_dev(ptr(dx), n_tok, n_in, ptr(dc), ptr(ds), stream())
    st = dev.sync_status(stream())
    return st, dc.cpu().numpy(), ds.cpu().numpy()


def test_quant_act_f32_bit_exact(dev):
    rng = np.random.default_rng(1)
    for n_tok, n_in in [(1, 896), (3, 33), (5, 4864), (2, 300), (7, 1536)]:
        x = rng.standard_normal((n_tok, n_in)).astype(np.float32)
        x[0, :32] = 0.0
        x[-1, 5] = 1e-20
        x[-1, 7] = -2.0e9
        st, c, s = quant_f32_gpu(dev, x)
        assert st == 0
        for r in range(n_tok):
            ost, oc, os_ = oracle.quant_act_f32(x[r])
            assert ost == 0
            assert (c[r] == oc).all() and (s[r] == os_).all(), (n_tok, n_in, r)


@pytest.mark.parametrize("t", [6, 8, 12, 14])
def test_f32_quantizer_rounding_edges(dev, t):
    """Activations built on the quantizer's rounding edges (tests/quant_edges.py: the element just
    below half a code unit, second roundings below 2^-9, the exponent's mantissa boundary, blocks
    outside the f32 fast form in the same waves as blocks inside it), over more than three passes
    of the streaming kernels' 128-block prologue: the device quantizer equals quant_act_f32, and
    the fused-quantizer GEMV equals the codes-input GEMV on the oracle's codes."""
    x = edge_blocks_f32(np.random.default_rng(31), normal_blocks=120)
    n_in = x.shape[0]
    assert n_in > 3 * 128 * 32
    ost, oc, os_ = oracle.quant_act_f32(x)
    assert ost == 0
    st, c, s = quant_f32_gpu(dev, x[None, :])
    assert st == 0
    assert (c[0] == oc).all() and (s[0] == os_).all()
    # The raw activation's largest blocks (up to 2^31) can overflow a row's output, which both
    # paths must refuse alike; a copy with every block above 2^8 scaled down by a power of two
    # (each block's rounding edges are relative to its own exponent, so they stay) must project.
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    shift = np.where(amax > 256.0, np.ceil(np.log2(np.maximum(amax, 1.0))) - 8, 0.0)
    tame = (xb * np.ldexp(1.0, -shift.astype(np.int64))[:, None]).astype(np.float32).reshape(-1)
    rng = synth.rng_for(7, t)
    for n_out in (64, 1536):
        w = dev.upload(t, synth.payload(t, rng, n_out, n_in), n_out, n_in)
        for name, xa in (("raw", x), ("tame", tame)):
            qst, qc, qs = oracle.quant_act_f32(xa)
            assert qst == 0
            # (device inputs held in names: a temporary's memory could be reused before the launch)
            dc, ds, dx = to_dev(qc), to_dev(qs), to_dev(xa)
            y = torch.empty(n_out, dtype=torch.float32, device="cuda")
            w.gemv_q8_dev(ptr(dc), ptr(ds), ptr(y), stream())
            st_codes = dev.sync_status(stream())
            yf = torch.empty(n_out, dtype=torch.float32, device="cuda")
            w.gemv_f32_dev(ptr(dx), ptr(yf), stream())
            st_f32 = dev.sync_status(stream())
            assert st_f32 == st_codes, (t, n_out, name)
            assert st_codes in ((0, 9) if name == "raw" else (0,)), (t, n_out, name, st_codes)
            if st_codes == 0:
                assert (yf.cpu().numpy() == y.cpu().numpy()).all(), (t, n_out, name)
        w.free()


def test_quant_act_f32_refusals(dev):
    x = np.ones((1, 64), np.float32)
    x[0, 40] = np.inf
    assert quant_f32_gpu(dev, x)[0] == 10
    x = np.ones((1, 64), np.float32)
    x[0, 3] = 3e9
    x[0, 50] = np.nan
    assert quant_f32_gpu(dev, x)[0] == 11  # the earlier element decides
    x = np.full((1, 32), 2147483520.0, np.float32)  # code 64 * 2^57 leaves i64
    assert quant_f32_gpu(dev, x)[0] == 7
    assert quant_f32_gpu(dev, np.ones((1, 64), np.float32))[0] == 0  # status was cleared


def test_quant_act_q32_reference_kats(dev):
    # chart/tests.rs:397-415
    q = dev.quant_act([3, 130, -3])
    assert q.codes.tolist() == [2, 65, -2] and q.scales.tolist() == [2]
    assert dev.quant_act([(1 << 63) - 1] * 32) is None
    q = dev.quant_act([-(1 << 63)] * 32)
    assert q.scales.tolist() == [1 << 57] and (q.codes == -64).all()
    q = dev.quant_act([127 << 56] * 32)
    assert (q.codes == 127).all() and q.scales.tolist() == [1 << 56]
    rng = np.random.default_rng(2)
    for seed in range(4):
        x = (rng.integers(-(1 << 62), 1 << 62, size=203) >> rng.integers(0, 60, size=203)).astype(np.int64)
        x[:32] = 0
        q = dev.quant_act(x)
        st, oc, os_ = oracle.quant_act(x)
        assert st == 0 and (q.codes == oc).all() and (q.scales == os_).all()


# ---- GEMV ------------------------------------------------------------------------------------

def test_gemv_golden_fixtures(dev):
    n = 0
    for c in golden_cases():
        w = dev.upload(c["t"], c["raw"], c["rows"], c["n_in"])
        y, dots = gemv_q8(dev, w, c["codes"], c["scales"], dots=True)
        assert (dots == c["dots"]).all(), (c["kind"], c["t"], c["n_in"])
        st, absdot = oracle.row_absdot(c["t"], c["raw"], c["rows"], c["n_in"], c["codes"], c["scales"])
        assert_close(y, c["y"], absdot, f"{c['kind']} t{c['t']} K{c['n_in']}")
        if c["xf"] is not None:
            yf = torch.empty(c["rows"], dtype=torch.float32, device="cuda")
            dx = to_dev(c["xf"])
            w.gemv_f32_dev(ptr(dx), ptr(yf), stream())
            assert dev.sync_status(stream()) == 0
            assert (yf.cpu().numpy() == y).all()  # fused quantizer == pre-quantized path
        w.free()
        n += 1
    assert n >= 40


@pytest.mark.parametrize("t", [6, 8, 10, 11, 12, 14])
@pytest.mark.parametrize("n_out,n_in", [(4864, 896), (896, 4864), (128, 896), (333, 1536), (37, 8960), (5, 100),
                                         (301, 300), (2001, 576), (7, 32768), (9, 20000)])
def test_gemv_config_shapes(dev, t, n_out, n_in):
    rng = synth.rng_for(1, t * 1000 + n_in)
    raw = synth.payload(t, rng, n_out, n_in)
    x = synth.activations(rng, n_in)
    st, codes, scales = oracle.quant_act_f32(x)
    assert st == 0
    w = dev.upload(t, raw, n_out, n_in)
    y, dots = gemv_q8(dev, w, codes, scales, dots=True)
    # exact oracle on every row for the small shapes, a row sample for the big ones
    rows = np.arange(n_out) if n_out * n_in <= 1_000_000 else np.unique(rng.integers(0, n_out, 64))
    rb = synth.row_bytes(t, n_in)
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
    st, yref = oracle.matvec_q8act(t, sub, len(rows), n_in, codes, scales)
    assert st == 0
    st, absdot = oracle.row_absdot(t, sub, len(rows), n_in, codes, scales)
    assert_close(y[rows], yref, absdot, f"t{t} {n_out}x{n_in}")
    for i, r in enumerate(rows[:16]):
        st, od, _ = oracle.block_dots(t, sub[i * rb:(i + 1) * rb], n_in, codes)
        assert (dots[r] == od).all(), (t, n_out, n_in, r)
    # fused f32 path is the same arithmetic
    yf = torch.empty(n_out, dtype=torch.float32, device="cuda")
    dx = to_dev(x)
    w.gemv_f32_dev(ptr(dx), ptr(yf), stream())
    assert dev.sync_status(stream()) == 0
    assert (yf.cpu().numpy() == y).all()
    w.free()


def test_gemv_vocab_head_q6_k_and_q8_0(dev):
    # config 2: 151936 x 896; exact oracle on a row sample, all rows finite and deterministic.
    for t in (14, 8):
        rng = synth.rng_for(2, t)
        n_out, n_in = 151936, 896
        raw = synth.payload(t, rng, n_out, n_in)
        x = synth.activations(rng, n_in)
        st, codes, scales = oracle.quant_act_f32(x)
        w = dev.upload(t, raw, n_out, n_in)
        y1 = gemv_q8(dev, w, codes, scales)
        y2 = gemv_q8(dev, w, codes, scales)
        assert (y1 == y2).all() and np.isfinite(y1).all()
        rows = np.unique(np.concatenate([[0, 1, n_out - 1], rng.integers(0, n_out, 200)]))
        rb = synth.row_bytes(t, n_in)
        sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
        st, yref = oracle.matvec_q8act(t, sub, len(rows), n_in, codes, scales)
        st2, absdot = oracle.row_absdot(t, sub, len(rows), n_in, codes, scales)
        assert st == 0 and st2 == 0
        assert_close(y1[rows], yref, absdot, f"head t{t}")
        w.free()


def test_gemv_linearity_full_size(dev):
    # size-independent property at a full config size: W(x) for codes c and the same codes with
    # every block scale doubled gives exactly 2x (power-of-two scales are exact in f32).
    rng = synth.rng_for(4, 7)
    raw = synth.payload(12, rng, 8960, 1536)
    x = synth.activations(rng, 1536)
    st, codes, scales = oracle.quant_act_f32(x)
    w = dev.upload(12, raw, 8960, 1536)
    y1 = gemv_q8(dev, w, codes, scales)
    y2 = gemv_q8(dev, w, codes, scales * 2)
    assert (y2 == 2 * y1).all()
    w.free()


def rows_vs_oracle(t, raw, n_in, x, y, what, max_rows=2048):
    """y (one projection's outputs for f32 input x) within the contract of the oracle, on every row
    up to max_rows and a sample past them."""
    n_out = y.shape[0]
    rows = np.arange(n_out) if n_out <= max_rows else np.unique(
        np.concatenate([np.arange(64), np.random.default_rng(n_out).integers(0, n_out, max_rows)]))
    rb = synth.row_bytes(t, n_in)
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
    st, codes, scales = oracle.quant_act_f32(x)
    assert st == 0
    st, yref = oracle.matvec_q8act(t, sub, len(rows), n_in, codes, scales)
    st2, absdot = oracle.row_absdot(t, sub, len(rows), n_in, codes, scales)
    assert st == 0 and st2 == 0
    assert_close(np.asarray(y)[rows], yref, absdot, what)


def test_grouped_plan_matches_single_launches(dev):
    """A table plan (more than four parts) of configs[1]-shaped Q4_K projections, and the same
    projections launched one by one, each within the contract of the oracle.  A table plan keeps
    whole super-blocks where a single launch of a small projection cuts sub-block pairs, so the two
    forms meet through the oracle rather than bit for bit."""
    rng = synth.rng_for(1, 99)
    shapes = [(896, 896), (128, 896), (128, 896), (896, 896), (4864, 896), (4864, 896), (896, 4864)]
    ws, xs, ys, singles, raws, xnp = [], [], [], [], [], []
    for n_out, n_in in shapes:
        raw = synth.payload(12, rng, n_out, n_in)
        w = dev.upload(12, raw, n_out, n_in)
        xa = synth.activations(rng, n_in)
        x = to_dev(xa)
        y = torch.zeros(n_out, dtype=torch.float32, device="cuda")
        ys1 = torch.zeros(n_out, dtype=torch.float32, device="cuda")
        w.gemv_f32_dev(ptr(x), ptr(ys1), stream())
        ws.append(w), xs.append(x), ys.append(y), singles.append(ys1), raws.append(raw), xnp.append(xa)
    plan = chart.GemvPlan(dev, ws, [ptr(x) for x in xs], [ptr(y) for y in ys])
    for _ in range(3):
        plan.run(stream())
    assert dev.sync_status(stream()) == 0
    for i, ((n_out, n_in), y, s) in enumerate(zip(shapes, ys, singles)):
        rows_vs_oracle(12, raws[i], n_in, xnp[i], y.cpu().numpy(), f"plan part {i}")
        rows_vs_oracle(12, raws[i], n_in, xnp[i], s.cpu().numpy(), f"single {i}")
    plan.free()
    for w in ws:
        w.free()


def _plan_vs_singles(dev, t, shapes, seed):
    """A plan's outputs equal single launches bit for bit, but for the Q4_K parts of a table plan
    (more than four parts): single launches of small projections cut sub-block pairs where a table
    plan keeps whole super-blocks, so those parts meet through the oracle (both forms within its
    contract).  t is one ggml type for every part, or a list with one type per shape (a mixed-type
    plan)."""
    rng = synth.rng_for(5, seed)
    types = t if isinstance(t, list) else [t] * len(shapes)
    ws, xs, ys, singles, raws, xnp = [], [], [], [], [], []
    for (n_out, n_in), t in zip(shapes, types):
        raw = synth.payload(t, rng, n_out, n_in)
        w = dev.upload(t, raw, n_out, n_in)
        xa = synth.activations(rng, n_in)
        x = to_dev(xa)
        y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
        ys1 = torch.zeros(n_out, dtype=torch.float32, device="cuda")
        w.gemv_f32_dev(ptr(x), ptr(ys1), stream())
        ws.append(w), xs.append(x), ys.append(y), singles.append(ys1), raws.append(raw), xnp.append(xa)
    plan = chart.GemvPlan(dev, ws, [ptr(x) for x in xs], [ptr(y) for y in ys])
    for _ in range(2):
        plan.run(stream())
    assert dev.sync_status(stream()) == 0
    table = len(shapes) > 4
    for i, (y, s1) in enumerate(zip(ys, singles)):
        if table and types[i] == 12:
            n_in = shapes[i][1]
            rows_vs_oracle(12, raws[i], n_in, xnp[i], y.cpu().numpy(), f"plan part {i} {shapes[i]}")
            rows_vs_oracle(12, raws[i], n_in, xnp[i], s1.cpu().numpy(), f"single {i} {shapes[i]}")
        else:
            assert torch.equal(y, s1), (t, i, shapes[i])
    plan.free()
    for w in ws:
        w.free()


@pytest.mark.parametrize("t", [8, 12, 14])
def test_plan_many_small_parts(dev, t):
    # one-tile parts get one wave each: workgroups serve up to 8 parts (8 activations in LDS),
    # mixed K, ragged rows, and trailing idle waves in the last workgroup
    shapes = [(3 + i % 5, (96, 300, 896, 1024)[i % 4]) for i in range(61)]
    _plan_vs_singles(dev, t, shapes, 10 + t)


@pytest.mark.parametrize("t", [8, 12])
def test_plan_activation_budget_padding(dev, t):
    # consecutive one-wave parts with K = 4864 overflow a workgroup's activation budget after two:
    # the next part starts a new workgroup and the skipped waves stay idle
    shapes = []
    for i in range(12):
        shapes += [(2, 4864), (5, 896)] if i % 3 == 0 else [(2, 4864)]
    _plan_vs_singles(dev, t, shapes, 30 + t)


def test_upload_refusals(dev):
    raw = synth.payload(8, synth.rng_for(0, 1), 4, 64)
    with pytest.raises(chart.MatvecError) as e:
        dev.upload(8, raw[:-1], 4, 64)
    assert e.value.kind == "ShortPayload"
    with pytest.raises(chart.MatvecError) as e:
        dev.upload(3, raw, 4, 64)
    assert e.value.kind == "UnsupportedQuant"
    for t, off in ((8, 34), (6, 22), (12, 146), (14, 210 + 208)):
        raw = synth.payload(t, synth.rng_for(0, t), 3, 256)
        raw[off:off + 2] = [0x00, 0x7C]  # +inf scale in a later block
        with pytest.raises(chart.MatvecError) as e:
            dev.upload(t, raw, 3, 256)
        assert e.value.kind == "NonFiniteScale"


def test_host_forms_mirror_reference_interface(dev):
    rng = synth.rng_for(0, 5)
    raw = synth.payload(12, rng, 40, 512)
    x = (rng.integers(-2048, 2048, size=512)).astype(np.int64)
    q = chart.quant_act(x)
    st, oc, os_ = oracle.quant_act(x)
    assert (q.codes == oc).all() and (q.scales == os_).all()
    y = chart.matvec_q8act(12, raw, 40, 512, q)
    st, yref = oracle.matvec_q8act(12, raw, 40, 512, oc, os_)
    st2, absdot = oracle.row_absdot(12, raw, 40, 512, oc, os_)
    assert_close(y, yref, absdot, "host matvec")
    with pytest.raises(chart.MatvecError) as e:
        chart.matvec_q8act(12, raw, 40, 256, q)
    assert e.value.kind == "ShapeMismatch"
    qs = [chart.quant_act(rng.integers(-5000, 5000, size=512).astype(np.int64)) for _ in range(5)]
    Y = chart.matmat_q8act(12, raw, 40, 512, qs)
    for c, qc in enumerate(qs):
        st, yc = oracle.matvec_q8act(12, raw, 40, 512, qc.codes, qc.scales)
        st2, ad = oracle.row_absdot(12, raw, 40, 512, qc.codes, qc.scales)
        assert_close(Y[c], yc, ad, f"host matmat col {c}")


# ---- GEMM ------------------------------------------------------------------------------------

def gemm_check(dev, t, n_out, n_in, n_tok, sample_cols=None, seed=0):
    rng = synth.rng_for(3, seed * 100 + t)
    raw = synth.payload(t, rng, n_out, n_in)
    x = synth.activations(rng, n_in, n_tok).reshape(n_tok, n_in)
    w = dev.upload(t, raw, n_out, n_in)
    dx = to_dev(x)
    y = torch.full((n_tok, n_out), float("nan"), dtype=torch.float32, device="cuda")
    w.gemm_f32_dev(ptr(dx), n_tok, ptr(y), stream())
    assert dev.sync_status(stream()) == 0
    Y = y.cpu().numpy()
    assert np.isfinite(Y).all()
    cols = range(n_tok) if sample_cols is None else sample_cols
    rows = np.arange(n_out) if n_out <= 1024 else np.unique(rng.integers(0, n_out, 96))
    rb = synth.row_bytes(t, n_in)
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
    for c in cols:
        st, codes, scales = oracle.quant_act_f32(x[c])
        st, yref = oracle.matvec_q8act(t, sub, len(rows), n_in, codes, scales)
        st2, absdot = oracle.row_absdot(t, sub, len(rows), n_in, codes, scales)
        assert st == 0 and st2 == 0
        assert_close(Y[c, rows], yref, absdot, f"gemm t{t} {n_out}x{n_in} N{n_tok} col {c}")
    # deterministic
    y2 = torch.empty_like(y)
    w.gemm_f32_dev(ptr(dx), n_tok, ptr(y2), stream())
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    w.free()
    return Y


@pytest.mark.parametrize("t", [6, 8, 10, 11, 12, 14])
@pytest.mark.parametrize("n_out,n_in,n_tok", [(64, 256, 8), (96, 300, 33), (200, 896, 130), (33, 64, 2)])
def test_gemm_small_shapes(dev, t, n_out, n_in, n_tok):
    gemm_check(dev, t, n_out, n_in, n_tok)


@pytest.mark.parametrize("t", [6, 8, 12])
@pytest.mark.parametrize("n_out,n_in", [(4864, 896), (896, 4864), (8960, 1536), (1536, 8960)])
def test_gemm_config3_shapes(dev, t, n_out, n_in):
    gemm_check(dev, t, n_out, n_in, 512, sample_cols=[0, 1, 127, 128, 255, 300, 511])


def test_gemm_q6_k_config4_shapes(dev):
    gemm_check(dev, 14, 256, 1536, 512, sample_cols=[0, 200, 511])
    gemm_check(dev, 14, 1536, 8960, 512, sample_cols=[0, 511])
    # 280 four-wave tiles on 256 CUs: served by the 2-wave kernel
    gemm_check(dev, 14, 8960, 1536, 512, sample_cols=[0, 300, 511])


@pytest.mark.parametrize("t,n_out,n_in", [(14, 8960, 1536), (8, 8960, 1536), (14, 1536, 8960),
                                          (8, 4864, 896), (12, 8960, 1536), (14, 256, 1536)])
def test_gemm_first_call_after_other_kernels(dev, t, n_out, n_in):
    """Every LDS ring slot holds this stage's slice before any wave reads it, whatever the CUs ran
    before: right after GEMMs of another type and shape (their data left in LDS), the first call
    equals the next calls bit for bit and the oracle.  Covers the three workgroup forms at N = 512
    (2 waves x 2 slots for 280-tile grids, 2 x 4 for small grids, 4 x 4 otherwise)."""
    n_tok = 512
    rng = synth.rng_for(8, t * 7 + n_out)
    ot = 12 if t != 12 else 14
    w_o = dev.upload(ot, synth.payload(ot, rng, 2048, 2048), 2048, 2048)
    x_o = torch.randn(n_tok, 2048, device="cuda")
    y_o = torch.empty((n_tok, 2048), dtype=torch.float32, device="cuda")
    raw = synth.payload(t, rng, n_out, n_in)
    x = synth.activations(rng, n_in, n_tok).reshape(n_tok, n_in)
    w = dev.upload(t, raw, n_out, n_in)
    dx = to_dev(x)
    ys = [torch.full((n_tok, n_out), float("nan"), dtype=torch.float32, device="cuda") for _ in range(3)]
    for _ in range(3):
        w_o.gemm_f32_dev(ptr(x_o), n_tok, ptr(y_o), stream())
    for y in ys:  # queued right behind the other GEMMs, no synchronisation in between
        w.gemm_f32_dev(ptr(dx), n_tok, ptr(y), stream())
    assert dev.sync_status(stream()) == 0
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[1], ys[2])
    Y = ys[0].cpu().numpy()
    rows = np.unique(rng.integers(0, n_out, 128))
    rb = synth.row_bytes(t, n_in)
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
    for c in (0, 77, 300, 511):
        st, codes, scales = oracle.quant_act_f32(x[c])
        st, yref = oracle.matvec_q8act(t, sub, len(rows), n_in, codes, scales)
        st2, absdot = oracle.row_absdot(t, sub, len(rows), n_in, codes, scales)
        assert_close(Y[c, rows], yref, absdot, f"first call t{t} {n_out}x{n_in} col {c}")
    w.free()
    w_o.free()


def test_gemm_n1_equals_gemv_within_tolerance(dev):
    rng = synth.rng_for(3, 77)
    for t in (8, 12, 14):
        raw = synth.payload(t, rng, 300, 896)
        x = synth.activations(rng, 896)
        w = dev.upload(t, raw, 300, 896)
        dx = to_dev(x.reshape(1, -1))
        y = torch.empty((1, 300), dtype=torch.float32, device="cuda")
        w.gemm_f32_dev(ptr(dx), 1, ptr(y), stream())
        assert dev.sync_status(stream()) == 0
        st, codes, scales = oracle.quant_act_f32(x)
        st, yref = oracle.matvec_q8act(t, raw, 300, 896, codes, scales)
        st2, absdot = oracle.row_absdot(t, raw, 300, 896, codes, scales)
        assert_close(y.cpu().numpy()[0], yref, absdot, f"gemm N=1 t{t}")
        w.free()


def test_mfma_probe_within_published_peaks(dev):
    """The MFMA-only probe must report a positive rate no higher than the dense peak of its
    instruction (a rate above the peak would mean the compiler dropped MFMAs from the loop)."""
    i8 = dev.probe_mfma_peak(0)
    f16 = dev.probe_mfma_peak(1)
    assert 0.0 < i8 <= 5000.0 * 1.05, i8
    assert 0.0 < f16 <= 2500.0 * 1.05, f16
    with pytest.raises(chart.MatvecError):
        dev.probe_mfma_peak(2)


@pytest.mark.parametrize("t", [6, 8, 10, 11, 12, 14])
@pytest.mark.parametrize("n_out,n_in,n_tok", [(96, 301, 5), (130, 8960, 70), (64, 20000, 3), (256, 1536, 129)])
def test_gemm_codes_input_equals_f32_input(dev, t, n_out, n_in, n_tok):
    """The codes-input GEMM (quantizer output handed over) equals the f32-input GEMM bit for bit:
    both build the same f16 operand from the same codes.  Covers bytewise code rows (n_in % 4 != 0),
    and the operand pass's 256-thread form and its 1024-thread forms of 2 and 4 register rounds
    (K = 8960, 20000); a few columns are checked against the oracle."""
    rng = synth.rng_for(3, 4000 + t + n_in)
    raw = synth.payload(t, rng, n_out, n_in)
    x = synth.activations(rng, n_in, n_tok).reshape(n_tok, n_in)
    w = dev.upload(t, raw, n_out, n_in)
    dx = to_dev(x)
    codes = torch.empty((n_tok, n_in), dtype=torch.int8, device="cuda")
    scales = torch.empty((n_tok, -(-n_in // 32)), dtype=torch.int64, device="cuda")
    dev.quant_act_f32_dev(ptr(dx), n_tok, n_in, ptr(codes), ptr(scales), stream())
    y1 = torch.full((n_tok, n_out), float("nan"), dtype=torch.float32, device="cuda")
    y2 = torch.full((n_tok, n_out), float("nan"), dtype=torch.float32, device="cuda")
    w.gemm_f32_dev(ptr(dx), n_tok, ptr(y1), stream())
    w.gemm_q8_dev(ptr(codes), ptr(scales), n_tok, ptr(y2), stream())
    assert dev.sync_status(stream()) == 0
    assert torch.isfinite(y1).all()
    assert torch.equal(y1, y2)
    Y = y2.cpu().numpy()
    for c in sorted({0, n_tok - 1}):
        st, cq, sq = oracle.quant_act_f32(x[c])
        st, yref = oracle.matvec_q8act(t, raw, n_out, n_in, cq, sq)
        st2, absdot = oracle.row_absdot(t, raw, n_out, n_in, cq, sq)
        assert st == 0 and st2 == 0
        assert_close(Y[c], yref, absdot, f"gemm codes t{t} {n_out}x{n_in} col {c}")
    w.free()


def test_mixed_type_plan_matches_single_launches(dev):
    """A Q4_K_M-style token (Q4_K and Q6_K projections, plus Q8_0 parts) in one mixed-type launch:
    every part's output is bit-identical to its own single-type launch."""
    parts = [(12, 1536, 1536), (12, 256, 1536), (14, 256, 1536), (12, 1536, 1536), (12, 8960, 1536),
             (14, 1536, 8960), (12, 1536, 8960), (8, 300, 896), (14, 5000, 1536), (8, 77, 7680),
             (12, 129, 300), (14, 33, 256)]
    _plan_vs_singles(dev, [t for t, _, _ in parts], [(n, k) for _, n, k in parts], 91)


def test_mixed_type_plan_with_q2_k_q3_k(dev):
    """Q2_K and Q3_K parts beside Q4_K / Q6_K / Q8_0 ones in one mixed-type launch (ragged widths
    included): each part's output equals its own single-type launch bit for bit."""
    parts = [(10, 1536, 1536), (11, 256, 1536), (12, 256, 1536), (14, 300, 896), (11, 77, 300),
             (10, 33, 4864), (8, 129, 896)]
    _plan_vs_singles(dev, [t for t, _, _ in parts], [(n, k) for _, n, k in parts], 92)


@pytest.mark.parametrize("t", [10, 11])
def test_plan_q2_k_q3_k_single_type(dev, t):
    """Single-type argument plans (up to four parts) and table plans of Q2_K / Q3_K projections."""
    _plan_vs_singles(dev, t, [(896, 896), (128, 896), (4864, 896)], 93 + t)
    _plan_vs_singles(dev, t, [(896, 896), (128, 896), (128, 896), (896, 896), (4864, 896), (896, 4864)], 95 + t)


def test_mixed_type_plan_refuses_rows_past_the_stream_tile(dev):
    """Mixed types need the streaming kernel: a Q8_0 part with K = 8192 (8704-byte rows) is refused."""
    rng = synth.rng_for(5, 92)
    w1 = dev.upload(12, synth.payload(12, rng, 64, 1536), 64, 1536)
    w2 = dev.upload(8, synth.payload(8, rng, 64, 8192), 64, 8192)
    x1, x2 = to_dev(synth.activations(rng, 1536)), to_dev(synth.activations(rng, 8192))
    y1 = torch.zeros(64, dtype=torch.float32, device="cuda")
    y2 = torch.zeros(64, dtype=torch.float32, device="cuda")
    with pytest.raises(chart.MatvecError) as ei:
        chart.GemvPlan(dev, [w1, w2], [ptr(x1), ptr(x2)], [ptr(y1), ptr(y2)])
    assert ei.value.status == 21  # AH_ERR_INVALID_ARG
    w1.free()
    w2.free()


@pytest.mark.parametrize("codes_input", [False, True])
def test_gemm_group_equals_single_projections(dev, codes_input):
    """One operand pass shared by q/k/v-like parts of mixed types (gemm_q8_0_group's shared pack,
    kern/gemm.rs:799-818): each part's output is bit-identical to its single-projection GEMM."""
    n_in, n_tok = 1536, 129
    shapes = [(12, 1536), (12, 256), (14, 256), (8, 300), (12, 0), (14, 4000)]
    rng = synth.rng_for(6, 31 + codes_input)
    x = to_dev(synth.activations(rng, n_in, n_tok).reshape(n_tok, n_in))
    codes = torch.empty((n_tok, n_in), dtype=torch.int8, device="cuda")
    scales = torch.empty((n_tok, n_in // 32), dtype=torch.int64, device="cuda")
    dev.quant_act_f32_dev(ptr(x), n_tok, n_in, ptr(codes), ptr(scales), stream())
    ws, ys, singles = [], [], []
    for t, n_out in shapes:
        w = dev.upload(t, synth.payload(t, rng, n_out, n_in), n_out, n_in)
        y = torch.full((n_tok, max(n_out, 1)), float("nan"), dtype=torch.float32, device="cuda")
        y1 = torch.full((n_tok, max(n_out, 1)), float("nan"), dtype=torch.float32, device="cuda")
        if codes_input:
            w.gemm_q8_dev(ptr(codes), ptr(scales), n_tok, ptr(y1), stream())
        else:
            w.gemm_f32_dev(ptr(x), n_tok, ptr(y1), stream())
        ws.append(w), ys.append(y), singles.append(y1)
    if codes_input:
        chart.gemm_group_q8_dev(dev, ws, ptr(codes), ptr(scales), n_tok, [ptr(y) for y in ys], stream())
    else:
        chart.gemm_group_f32_dev(dev, ws, ptr(x), n_tok, [ptr(y) for y in ys], stream())
    assert dev.sync_status(stream()) == 0
    for (t, n_out), y, y1 in zip(shapes, ys, singles):
        if n_out:
            assert torch.isfinite(y).all(), (t, n_out)
            assert torch.equal(y, y1), (t, n_out)
        else:  # a part without rows writes nothing
            assert torch.isnan(y).all() and torch.isnan(y1).all()
    # parts must share n_in
    w_bad = dev.upload(12, synth.payload(12, rng, 64, 896), 64, 896)
    with pytest.raises(chart.MatvecError) as ei:
        chart.gemm_group_f32_dev(dev, [ws[0], w_bad], ptr(x), n_tok, [ptr(ys[0]), ptr(ys[1])], stream())
    assert ei.value.status == 21
    for w in ws + [w_bad]:
        w.free()


GROUP_LAYOUTS = [
    # configs[4] q/k/v at prefill size: two Q4_K parts in one launch, both split, then Q6_K
    (1536, 512, [(12, 1536), (12, 256), (14, 256)]),
    # configs[4] gate/up: two 280-tile Q4_K parts in one launch
    (1536, 512, [(12, 8960), (12, 8960)]),
    # a run of six Q4_K parts (two launches), an empty part inside it, ragged n_out whose
    # n_tok * n_out is odd (the scalar reduction path for the whole group)
    (896, 201, [(12, 100), (12, 0), (12, 257), (12, 64), (12, 896), (12, 33), (12, 128)]),
    # consecutive Q6_K parts of different split counts, then Q8_0 parts (one per launch)
    (2048, 300, [(14, 2048), (14, 96), (14, 520), (8, 700), (8, 64)]),
    # ten one-tile Q4_K parts, all split: three GEMM launches (4 + 4 + 2 parts) and two
    # reduction launches (8 + 2 parts)
    (2048, 64, [(12, 64 + 32 * i) for i in range(10)]),
    # alternating Q6_K / Q4_K parts in one mixed K-quant grid, ragged widths, then a fifth part
    (1536, 200, [(14, 300), (12, 700), (14, 64), (12, 1000), (14, 129)]),
]


@pytest.mark.parametrize("layout", range(len(GROUP_LAYOUTS)))
def test_gemm_group_runs_equal_single_projections(dev, layout):
    """Grouped prefill launches several parts of one type in one grid and reduces every split part
    in one pass; each part's output equals its single-projection GEMM bit for bit."""
    n_in, n_tok, shapes = GROUP_LAYOUTS[layout]
    rng = synth.rng_for(7, 50 + layout)
    x = to_dev(synth.activations(rng, n_in, n_tok).reshape(n_tok, n_in))
    ws, ys, singles = [], [], []
    for t, n_out in shapes:
        w = dev.upload(t, synth.payload(t, rng, n_out, n_in), n_out, n_in)
        y = torch.full((n_tok, max(n_out, 1)), float("nan"), dtype=torch.float32, device="cuda")
        y1 = torch.full((n_tok, max(n_out, 1)), float("nan"), dtype=torch.float32, device="cuda")
        w.gemm_f32_dev(ptr(x), n_tok, ptr(y1), stream())
        ws.append(w), ys.append(y), singles.append(y1)
    chart.gemm_group_f32_dev(dev, ws, ptr(x), n_tok, [ptr(y) for y in ys], stream())
    assert dev.sync_status(stream()) == 0
    for (t, n_out), y, y1 in zip(shapes, ys, singles):
        if n_out:
            assert torch.isfinite(y).all(), (t, n_out)
            assert torch.equal(y, y1), (t, n_out)
        else:
            assert torch.isnan(y).all() and torch.isnan(y1).all()
    for w in ws:
        w.free()
