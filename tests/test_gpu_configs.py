"""GPU parity of the grouped paths and of BASELINE configs[4]'s shapes against the CPU oracle.

Each part of a grouped launch (a GEMV plan, a grouped prefill) is compared with the oracle's exact
matvec_q8act on its own input, not with another HIP launch:

* a configs[1] layer (Qwen2.5-0.5B: q/o 896x896, k/v 128x896, gate/up 4864x896, down 896x4864,
  Q4_K) as one plan launch;
* configs[4] layers (Qwen2.5-1.5B, Q4_K_M mix: attn_v Q6_K, ffn_down Q6_K on llama.cpp's
  use_more_bits layers) as one mixed-type plan at N = 1 and as grouped prefill calls at N = 512;
* the configs[4] vocab head, Q6_K 151936x1536, at N = 1 and N = 512 (sampled rows and columns).

Bar: |y - y_ref| <= 1e-4 * sum|w*xhat| + 2^-32 per output (y_ref the exact Q32.32 contract).
"""
import numpy as np
import pytest

import oracle
from apeiron_amd import chart, synth

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-4
Q32 = 2.0 ** -32
Q5_0, Q8_0, Q4_K, Q6_K = 6, 8, 12, 14
CFG4_Q6K_DOWN = {0, 1, 2, 5, 8, 11, 14, 17, 20, 23, 24, 25, 26, 27}


def cfg4_layer(l):
    """configs[4] layer l: (name, type, n_out, n_in) in the engine's projection order."""
    return [("q", Q4_K, 1536, 1536), ("k", Q4_K, 256, 1536), ("v", Q6_K, 256, 1536),
            ("o", Q4_K, 1536, 1536), ("gate", Q4_K, 8960, 1536), ("up", Q4_K, 8960, 1536),
            ("down", Q6_K if l in CFG4_Q6K_DOWN else Q4_K, 1536, 8960)]


CFG1_LAYER = [("q", Q4_K, 896, 896), ("k", Q4_K, 128, 896), ("v", Q4_K, 128, 896),
              ("o", Q4_K, 896, 896), ("gate", Q4_K, 4864, 896), ("up", Q4_K, 4864, 896),
              ("down", Q4_K, 896, 4864)]


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


def sample_rows(rng, n_out, k=96):
    return np.arange(n_out) if n_out <= 1024 else np.unique(rng.integers(0, n_out, k))


def check_rows(t, raw, n_in, rows, x, y_rows, what):
    """y_rows (the GPU's outputs of `rows` for f32 input x) against the oracle."""
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


def plan_vs_oracle(dev, layer, seed):
    rng = synth.rng_for(4, seed)
    parts = []
    for name, t, n_out, n_in in layer:
        raw = synth.payload(t, rng, n_out, n_in)
        x = synth.activations(rng, n_in)
        parts.append((name, t, n_out, n_in, raw, x, dev.upload(t, raw, n_out, n_in), to_dev(x),
                      torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")))
    plan = chart.GemvPlan(dev, [p[6] for p in parts], [p[7].data_ptr() for p in parts],
                          [p[8].data_ptr() for p in parts])
    plan.run(stream())
    assert dev.sync_status(stream()) == 0
    for name, t, n_out, n_in, raw, x, w, dx, dy in parts:
        rows = sample_rows(rng, n_out)
        check_rows(t, raw, n_in, rows, x, dy.cpu().numpy()[rows], f"plan part {name} {n_out}x{n_in}")
    plan.free()
    for p in parts:
        p[6].free()


def test_config1_layer_plan_parts_vs_oracle(dev):
    """The headline token plan's parts (one configs[1] layer, one launch) each against the oracle,
    q and o 896x896 on every row."""
    plan_vs_oracle(dev, CFG1_LAYER, 1)


@pytest.mark.parametrize("layer", [0, 3])
def test_config4_layer_mixed_plan_vs_oracle(dev, layer):
    """A configs[4] layer's 7 projections (Q4_K with Q6_K attn_v, and ffn_down Q6_K on layer 0,
    Q4_K on layer 3) in one mixed-type plan launch, each part against the oracle."""
    plan_vs_oracle(dev, cfg4_layer(layer), 10 + layer)


@pytest.mark.parametrize("layer", [0, 3])
def test_config4_decode_stage_plans_vs_oracle(dev, layer):
    """The configs[4] decode stages as a token issues them: q/k/v (Q4_K, Q4_K, Q6_K: one mixed
    launch), o, gate/up, down.  Plans of at most 4 parts carry their descriptors in the kernel
    arguments (whole workgroups per part); every part against the oracle."""
    proj = cfg4_layer(layer)
    for g in ([0, 1, 2], [3], [4, 5], [6]):
        plan_vs_oracle(dev, [proj[i] for i in g], 20 + 10 * layer + g[0])


def test_argument_plan_limits_vs_oracle(dev):
    """Four parts (the most the kernel arguments carry) and five (the workgroup-table plan), mixed
    types and ragged shapes, every part against the oracle."""
    four = [("a", Q6_K, 300, 512), ("b", Q4_K, 7, 768), ("c", Q8_0, 1000, 96), ("d", Q4_K, 129, 256)]
    plan_vs_oracle(dev, four, 40)
    plan_vs_oracle(dev, four + [("e", Q6_K, 33, 1024)], 41)
    plan_vs_oracle(dev, [("s", Q8_0, 1, 32)], 42)
    # Q5_0 parts through the mixed-type kernel (argument and table plans) and alone
    q5 = [("q5a", Q5_0, 640, 896), ("q4", Q4_K, 100, 896), ("q5b", Q5_0, 33, 300), ("q6", Q6_K, 64, 512)]
    plan_vs_oracle(dev, q5, 43)
    plan_vs_oracle(dev, q5 + [("q5c", Q5_0, 5, 4864)], 44)
    plan_vs_oracle(dev, [("q5", Q5_0, 896, 896), ("q5k", Q5_0, 128, 896)], 45)


def test_qwen05b_q4_k_m_layer_with_q5_0_tensors(dev):
    """A Qwen2.5-0.5B layer in a mixed-quant checkpoint's style (its ffn_gate and attn_output are
    Q5_0 there, tests/gpu_gemv_match.rs:252-275; here every K = 896 tensor is Q5_0 and ffn_down
    Q6_K): one mixed plan at N = 1 and the grouped prefill at N = 300, every part against the
    oracle."""
    layer = [("q", Q5_0, 896, 896), ("k", Q5_0, 128, 896), ("v", Q5_0, 128, 896), ("o", Q5_0, 896, 896),
             ("gate", Q5_0, 4864, 896), ("up", Q5_0, 4864, 896), ("down", Q6_K, 896, 4864)]
    plan_vs_oracle(dev, layer, 46)
    rng = synth.rng_for(1, 4600)
    n_tok = 300
    x = synth.activations(rng, 896, n_tok)
    dx = to_dev(x)
    parts = [p for p in layer if p[3] == 896]
    raws = [synth.payload(t, rng, n, k) for _, t, n, k in parts]
    W = [dev.upload(t, r, n, k) for (_, t, n, k), r in zip(parts, raws)]
    ys = [torch.full((n_tok, n), float("nan"), dtype=torch.float32, device="cuda") for _, _, n, _ in parts]
    chart.gemm_group_f32_dev(dev, W, dx.data_ptr(), n_tok, [y.data_ptr() for y in ys], stream())
    assert dev.sync_status(stream()) == 0
    for (name, t, n, k), raw, y in zip(parts, raws, ys):
        Y = y.cpu().numpy()
        rows = sample_rows(rng, n, 64)
        for c in (0, 150, 299):
            check_rows(t, raw, k, rows, x[c], Y[c, rows], f"q5_0 layer {name} col {c}")
    for w in W:
        w.free()


@pytest.mark.parametrize("layer", [0, 3])
def test_config4_layer_prefill_groups_vs_oracle(dev, layer):
    """One configs[4] layer at N = 512 as the engine issues it: q/k/v grouped on one input, o,
    gate/up grouped, down; sampled rows x columns of every part against the oracle."""
    rng = synth.rng_for(4, 100 + layer)
    n_tok = 512
    proj = cfg4_layer(layer)
    groups = [[0, 1, 2], [3], [4, 5], [6]]
    W, raws = [], []
    for name, t, n_out, n_in in proj:
        raw = synth.payload(t, rng, n_out, n_in)
        raws.append(raw)
        W.append(dev.upload(t, raw, n_out, n_in))
    for g in groups:
        n_in = proj[g[0]][3]
        x = synth.activations(rng, n_in, n_tok)
        dx = to_dev(x)
        ys = [torch.full((n_tok, proj[i][2]), float("nan"), dtype=torch.float32, device="cuda") for i in g]
        chart.gemm_group_f32_dev(dev, [W[i] for i in g], dx.data_ptr(), n_tok, [y.data_ptr() for y in ys], stream())
        assert dev.sync_status(stream()) == 0
        for i, y in zip(g, ys):
            name, t, n_out, _ = proj[i]
            Y = y.cpu().numpy()
            rows = sample_rows(rng, n_out, 64)
            for c in (0, 63, 64, 200, 511):
                check_rows(t, raws[i], n_in, rows, x[c], Y[c, rows], f"prefill {name} col {c}")
    for w in W:
        w.free()


def test_config4_vocab_head_q6_k(dev):
    """The configs[4] head, Q6_K 151936x1536: N = 1 (GEMV) and N = 512 (GEMM), sampled."""
    rng = synth.rng_for(4, 999)
    n_out, n_in = 151936, 1536
    raw = synth.payload(Q6_K, rng, n_out, n_in)
    w = dev.upload(Q6_K, raw, n_out, n_in)
    rows = np.concatenate([np.arange(8), np.unique(rng.integers(0, n_out, 120)), np.arange(n_out - 8, n_out)])
    x1 = synth.activations(rng, n_in)
    y1 = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
    w.gemv_f32_dev(to_dev(x1).data_ptr(), y1.data_ptr(), stream())
    assert dev.sync_status(stream()) == 0
    check_rows(Q6_K, raw, n_in, rows, x1, y1.cpu().numpy()[rows], "head N=1")
    n_tok = 512
    x = synth.activations(rng, n_in, n_tok)
    y = torch.full((n_tok, n_out), float("nan"), dtype=torch.float32, device="cuda")
    w.gemm_f32_dev(to_dev(x).data_ptr(), n_tok, y.data_ptr(), stream())
    assert dev.sync_status(stream()) == 0
    Y = y.cpu().numpy()
    assert np.isfinite(Y).all()
    for c in (0, 127, 128, 333, 511):
        check_rows(Q6_K, raw, n_in, rows, x[c], Y[c, rows], f"head N=512 col {c}")
    del y
    w.free()
