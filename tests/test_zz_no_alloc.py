"""ah_gemm_f32_noalloc_dev (the GEMM entry point that allocates nothing) against ah_gemm_f32_dev,
through the C ABI: bit-identical outputs on two calls in a row, the second with a smaller input
(its fixed scratch keeps the first call's contents), and a clear refusal past its scratch."""
import ctypes

import numpy as np
import pytest

from apeiron_amd import chart, synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    d = chart.Device(0)
    yield d
    d.close()


def run(dev, fn, w, x):
    n_tok = x.shape[0]
    y = torch.full((n_tok, w.n_out), float("nan"), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    st = fn(dev.h, w.h, x.data_ptr(), n_tok, y.data_ptr(), s)
    assert st == 0, chart._lib.STATUS.get(st, st)
    assert dev.sync_status(s) == 0
    return y


@pytest.mark.parametrize("t,design", [(8, 0), (12, 0), (14, 0), (8, 2), (12, 2)])
def test_noalloc_gemm_equals_gemm(dev, t, design):
    """Every type's default design, and the int8 designs of Q8_0 and Q4_K (their codes, block
    factors and Q4_K's scaled code sums in the fixed scratch)."""
    dev.set_gemm_design(t, design)
    try:
        check_noalloc_equals_gemm(dev, t)
    finally:
        dev.set_gemm_design(t, chart.Device.GEMM_AUTO)


def check_noalloc_equals_gemm(dev, t):
    L = dev.lib
    cap = ctypes.c_size_t(0)
    assert L.ah_gemm_noalloc_scratch_bytes(ctypes.byref(cap)) == 0 and cap.value == 64 << 20
    rng = synth.rng_for(7, t)
    # a split-K shape at N = 512 (partials in the scratch), then a smaller call on another weight
    shapes = [(1536, 8960, 512), (300, 896, 37)]
    outs = []
    for n_out, n_in, n_tok in shapes:
        raw = synth.payload(t, rng, n_out, n_in)
        w = dev.upload(t, raw, n_out, n_in)
        x = torch.from_numpy(synth.activations(rng, n_in, n_tok).reshape(n_tok, n_in)).cuda()
        x[n_tok // 2] *= torch.exp2(torch.arange(n_in, device="cuda") // 32 * 40.0 / (n_in // 32) - 20)
        y_na = run(dev, L.ah_gemm_f32_noalloc_dev, w, x)
        y_ref = run(dev, L.ah_gemm_f32_dev, w, x)
        assert torch.equal(y_na, y_ref), (t, n_out, n_in, n_tok)
        outs.append((w, x, y_na))
    # the first shape again after the smaller call: same result
    w, x, y0 = outs[0]
    assert torch.equal(run(dev, L.ah_gemm_f32_noalloc_dev, w, x), y0)
    for w, _, _ in outs:
        w.free()


def test_noalloc_gemm_refuses_past_its_scratch(dev):
    rng = synth.rng_for(7, 99)
    n_out, n_in, n_tok = 64, 8960, 4096  # operands alone: 4096 * 8960 * 3 bytes > 64 MiB
    w = dev.upload(8, synth.payload(8, rng, n_out, n_in), n_out, n_in)
    x = torch.zeros((n_tok, n_in), dtype=torch.float32, device="cuda")
    y = torch.zeros((n_tok, n_out), dtype=torch.float32, device="cuda")
    st = dev.lib.ah_gemm_f32_noalloc_dev(dev.h, w.h, x.data_ptr(), n_tok, y.data_ptr(), None)
    assert st == 24  # AH_ERR_SCRATCH_LIMIT, before anything is enqueued
    w.free()


@pytest.mark.parametrize("t", [10, 11])
def test_noalloc_gemm_q2_k_q3_k_route(dev, t):
    """The Q2_K / Q3_K prefill route (GEMV launches of four tokens' argument parts) through the
    no-alloc entry point equals the ordinary one bit for bit, on two calls in a row, the second
    with a smaller input."""
    L = dev.lib
    for n_out, n_in, n_tok in ((300, 896, 9), (64, 512, 3)):
        rng = synth.rng_for(12, t * 10 + n_tok)
        w = dev.upload(t, synth.payload(t, rng, n_out, n_in), n_out, n_in)
        x = torch.from_numpy(synth.activations(rng, n_in, n_tok).reshape(n_tok, n_in)).cuda()
        y1 = run(dev, L.ah_gemm_f32_dev, w, x)
        y2 = run(dev, L.ah_gemm_f32_noalloc_dev, w, x)
        assert torch.isfinite(y1).all() and torch.equal(y1, y2)
        w.free()


def test_noalloc_allocates_nothing(dev):
    """On a context that has never run an allocating GEMM: the no-alloc entry point leaves the
    device's free memory and the context's scratch exactly as they were, on the MFMA route (Q4_K),
    the dequantize-once tiles (Q3_K) and the per-token GEMV route (Q3_K, AH_GEMM_DESIGN_F16)."""
    L = dev.lib
    cases = [(12, 1536, 8960, 512, 0), (11, 896, 1536, 128, 0), (11, 300, 896, 9, 1)]
    # the kernels' code is loaded on first use: warm every route on the module's context first
    ws = {}
    for t, n_out, n_in, n_tok, design in cases:
        rng = synth.rng_for(13, t * 10 + design)
        raw = synth.payload(t, rng, n_out, n_in)
        x = torch.from_numpy(synth.activations(rng, n_in, n_tok).reshape(n_tok, n_in)).cuda()
        dev.set_gemm_design(t, design)
        w = dev.upload(t, raw, n_out, n_in)
        y_ref = run(dev, L.ah_gemm_f32_noalloc_dev, w, x)
        dev.set_gemm_design(t, 0)
        w.free()
        ws[(t, design)] = (raw, x, y_ref)
    fresh = chart.Device(0)
    try:
        W = {k: fresh.upload(k[0], ws[k][0], n_out, n_in) for (t, n_out, n_in, _, design) in cases
             for k in [(t, design)]}
        ys = {k: torch.empty((ws[k][1].shape[0], W[k].n_out), dtype=torch.float32, device="cuda") for k in W}
        probe = torch.zeros(W[(11, 1)].n_out, dtype=torch.float32, device="cuda")
        W[(11, 1)].gemv_f32_dev(ws[(11, 1)][1].data_ptr(), probe.data_ptr(), None)  # the stream's first launch
        assert fresh.sync_status(None) == 0
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        sts = []
        for (t, design), w in W.items():
            fresh.set_gemm_design(t, design)
            x = ws[(t, design)][1]
            st = L.ah_gemm_f32_noalloc_dev(fresh.h, w.h, x.data_ptr(), x.shape[0], ys[(t, design)].data_ptr(), None)
            sts.append((st, fresh.sync_status(None)))
        torch.cuda.synchronize()
        free1 = torch.cuda.mem_get_info()[0]  # before any torch work that could grow its cache
        assert free1 == free0, (free0, free1)
        assert all(s == (0, 0) for s in sts), sts
        for k in W:
            assert torch.equal(ys[k], ws[k][2]), k
        held = ctypes.c_size_t(1)
        assert L.ah_ctx_scratch_bytes(fresh.h, ctypes.byref(held)) == 0 and held.value == 0
        for w in W.values():
            w.free()
    finally:
        fresh.close()
