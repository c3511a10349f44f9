"""GPU: the first refusal of a grouped call is the one separate calls joined left to right would
return -- projection, then column (token), then row.

* projections_q8act (chart/ffn.rs:905-924): "the first refusal in projection-then-row order";
* the column path runs proj_cols part by part (step/cols.rs:485-575), each matmat_q8act
  reporting its first failing column (kern/matmat.rs:134).

Each case puts an OutputOverflow (9) in an earlier projection and an AccumulatorOverflow (8) in
a later one at the same or an earlier (token, row): a key ordered token-major across parts would
report 8.  The expected codes are the oracle's.
"""
import numpy as np
import pytest

import oracle
from apeiron_amd import chart, synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q4_K, Q3_K = 12, 11
N_IN = 4096


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    d = chart.Device(0)
    yield d
    d.close()


def stream():
    return torch.cuda.current_stream().cuda_stream


def const_payload(t, n_out, d_bits):
    """Every weight the same: Q4_K d * 63 * 15 (sc 63, codes 15, dmin 0); Q3_K d * (-32) * (-4)
    (all-zero codes, masks and scales)."""
    nsb = n_out * N_IN // 256
    if t == Q4_K:
        blk = np.zeros((nsb, 144), np.uint8)
        blk[:, 0], blk[:, 1] = d_bits & 0xFF, d_bits >> 8
        blk[:, 4:16] = synth.pack_q4_k_scales(np.full((nsb, 8), 63, np.uint8), np.zeros((nsb, 8), np.uint8))
        blk[:, 16:] = 0xFF
    else:
        blk = np.zeros((nsb, 110), np.uint8)
        blk[:, 108], blk[:, 109] = d_bits & 0xFF, d_bits >> 8
    return blk.reshape(-1)


SMALL, BIG = 0x1400, 0x7BFF  # f16 2^-10 and 65504


def contract(t, raws, n_out, codes, scales):
    """First refusal over parts, then tokens (the oracle per part and column)."""
    for raw in raws:
        for c in range(codes.shape[0]):
            st, _ = oracle.matvec_q8act(t, raw, n_out, N_IN, codes[c], scales[c])
            if st:
                return st
    return 0


@pytest.mark.parametrize("t,design", [(Q4_K, 0), (Q4_K, 3), (Q3_K, 0), (Q3_K, 1)])
def test_group_gemm_refusal_in_part_order(dev, t, design):
    n_out = 3
    top = (np.full(N_IN, 127, np.int8), np.full(N_IN // 32, 1 << 56, np.int64))
    low = (np.full(N_IN, 1, np.int8), np.full(N_IN // 32, 1 << 20, np.int64))
    raws = {k: const_payload(t, n_out, b) for k, b in (("small", SMALL), ("big", BIG))}
    W = {k: dev.upload(t, r, n_out, N_IN) for k, r in raws.items()}
    dev.set_gemm_design(t, design)
    try:
        for order in (("small", "big"), ("big", "small")):
            for toks in ((top,), (low, top), (top, low, low)):
                codes = np.stack([q[0] for q in toks])
                scales = np.stack([q[1] for q in toks])
                want = contract(t, [raws[k] for k in order], n_out, codes, scales)
                assert want in (8, 9)
                dc, ds = torch.from_numpy(codes).cuda(), torch.from_numpy(scales).cuda()
                ys = [torch.empty((len(toks), n_out), dtype=torch.float32, device="cuda") for _ in order]
                chart.gemm_group_q8_dev(dev, [W[k] for k in order], dc.data_ptr(), ds.data_ptr(), len(toks),
                                        [y.data_ptr() for y in ys], stream())
                assert dev.sync_status(stream()) == want, (order, len(toks))
    finally:
        dev.set_gemm_design(t, 0)
        for w in W.values():
            w.free()


@pytest.mark.parametrize("t", [Q4_K, Q3_K])
def test_gemv_plan_refusal_in_part_order(dev, t):
    """A decode plan over two projections of one input: part order, then row."""
    n_out = 3
    raws = {k: const_payload(t, n_out, b) for k, b in (("small", SMALL), ("big", BIG))}
    W = {k: dev.upload(t, r, n_out, N_IN) for k, r in raws.items()}
    x = torch.full((N_IN,), 2.0 ** 30, dtype=torch.float32, device="cuda")
    st, codes, scales = oracle.quant_act_f32(x.cpu().numpy())
    assert st == 0
    try:
        for order in (("small", "big"), ("big", "small")):
            want = contract(t, [raws[k] for k in order], n_out, codes[None], scales[None])
            assert want == (9 if order[0] == "small" else 8)
            ys = [torch.empty(n_out, dtype=torch.float32, device="cuda") for _ in order]
            plan = chart.GemvPlan(dev, [W[k] for k in order], [x.data_ptr()] * 2, [y.data_ptr() for y in ys])
            plan.run(stream())
            assert dev.sync_status(stream()) == want, order
            plan.free()
    finally:
        for w in W.values():
            w.free()
