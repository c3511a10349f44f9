#!/usr/bin/env python3
"""Benchmark of the quantized linear-layer path on one MI355X.

Headline: Q4_K GEMV decode, N = 1, over the Qwen2.5-0.5B
projection shapes.  One step is one token through a 24-layer stack of the seven projections
(q 896x896, k/v 128x896, o 896x896, gate/up 4864x896, down 896x4864), each an f32 N(0,1) input
quantized inside the kernel.  The weights of consecutive steps come from a rotating pool of
layer copies larger than 1 GiB, so every step streams its weights from HBM (the 256 MB
Infinity Cache is defeated), and the inputs are already resident in HBM.

Dispatch modes (``--mode``):
  token   (default) all 168 projections of a step in one grouped launch: the path's streaming
          rate.  The projections of a token are independent here because their callers
          (RMSNorm, attention, SwiGLU) are outside this path;
  engine  the reference engine's dispatch shape per layer: one grouped launch for q/k/v
          (shared input, chart/ffn.rs:925), o, one grouped launch for gate/up (shared input),
          down -- 4 dependent launches per layer, captured in a HIP graph per step window.  This
          is latency-bound (96 serialized kernels per token) and is reported beside the value.

Timing: the hot path first runs untimed for 150 ms (clock ramp-up of an idle GPU), then the W
warm-up steps, then the K timed steps between two synchronizations.

value = algorithmic bytes per step * steps / wall time (GB/s).  Algorithmic bytes per
projection = n_out * (weight bytes a correct kernel must read per row) + 4*n_in (f32 input)
+ 4*n_out (f32 output).

Also reported: the dominant kernel against the 8 TB/s HBM roofline (HIP events on the launch
stream), the N = 512 GEMMs of configs[3] against the 5.0 POPS dense int8 MFMA peak, and the
CPU baseline (the restated reference fast path, oracle/ah_cpu_fast.c, on this host's cores).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
CLOCK_WARMUP_S = 0.15  # untimed hot-path load before the warm-up steps (clock ramp-up)
INT8_PEAK_TOPS = 5000.0
F16_PEAK_TFLOPS = 2500.0  # dense f16 MFMA peak (the instruction the GEMM computes with)
LAYERS = 24
SHAPES = [("q", 896, 896), ("k", 128, 896), ("v", 128, 896), ("o", 896, 896),
          ("gate", 4864, 896), ("up", 4864, 896), ("down", 896, 4864)]
GEMM_SHAPES = [(4864, 896), (896, 4864), (8960, 1536), (1536, 8960)]
# Qwen2.5-1.5B architecture, Q4_K_M-style mix (Q6_K for attn_v, for ffn_down on
# llama.cpp's use_more_bits layers, and for the output head)
CFG4_LAYERS = 28
CFG4_Q6K_DOWN = {0, 1, 2, 5, 8, 11, 14, 17, 20, 23, 24, 25, 26, 27}


def cfg4_projections(synth):
    out = []
    for l in range(CFG4_LAYERS):
        out += [(synth.Q4_K, 1536, 1536), (synth.Q4_K, 256, 1536), (synth.Q6_K, 256, 1536),
                (synth.Q4_K, 1536, 1536), (synth.Q4_K, 8960, 1536), (synth.Q4_K, 8960, 1536),
                (synth.Q6_K if l in CFG4_Q6K_DOWN else synth.Q4_K, 1536, 8960)]
    out.append((synth.Q6_K, 151936, 1536))  # output head
    return out


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def proj_bytes(synth, t, n_out, n_in):
    return n_out * synth.needed_row_bytes(t, n_in) + 4 * n_in + 4 * n_out


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_stream_q4k_config1_token.md")


def measured_traffic():
    """HBM bytes per token-plan launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs
    (copy-calibrated; the counters cannot be read from inside this process), or None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--mode", choices=["engine", "token"], default="token")
    ap.add_argument("--pool-gib", type=float, default=1.1)
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-heads", action="store_true", help="skip configs[0] and configs[2]")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--cpu-threads", type=int, default=8)
    ap.add_argument("--only", choices=["gemv", "gemm", "copy", "config4", "heads"], default=None)
    ap.add_argument("--no-config4", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build has no "
              "multi-GPU path (a projection would shard by output rows, one row range per GPU, "
              "with no collective on the GEMV or GEMM itself).", file=sys.stderr)
        return 2

    import torch

    from apeiron_amd import chart, synth

    dev = chart.Device(0)
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    t = synth.Q4_K
    result: dict = {}

    if args.only == "copy":
        # calibration for the FETCH_SIZE / WRITE_SIZE counters: a plain 256 MiB copy
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": a.numel()}))
        return 0

    # ---- config 1: weight pool ------------------------------------------------------------
    layer_bytes_stored = sum(n * synth.row_bytes(t, k) for _, n, k in SHAPES)
    n_sets = max(LAYERS + 8, int(args.pool_gib * (1 << 30) // layer_bytes_stored) + 1)
    n_unique = 4
    log(f"[bench] pool: {n_sets} layer copies x {layer_bytes_stored / 1e6:.2f} MB = "
        f"{n_sets * layer_bytes_stored / 2**30:.2f} GiB")
    host_layers = []
    for u in range(n_unique):
        rng = synth.rng_for(1, 100 + u)
        host_layers.append({name: synth.payload(t, rng, n, k) for name, n, k in SHAPES})
    rng = synth.rng_for(1, 1)
    xin = {name: torch.from_numpy(synth.activations(rng, k)).cuda() for name, _, k in SHAPES}
    layers = []
    for i in range(n_sets):
        src = host_layers[i % n_unique]
        layers.append({name: dev.upload(t, src[name], n, k) for name, n, k in SHAPES})
    outs = {name: torch.zeros(n, dtype=torch.float32, device="cuda") for name, n, _ in SHAPES}
    step_bytes = LAYERS * sum(proj_bytes(synth, t, n, k) for _, n, k in SHAPES)
    x_attn, x_ffn = xin["q"], xin["gate"]

    def ptr(x):
        return x.data_ptr()

    # ---- config 1: dispatch ---------------------------------------------------------------
    plans = []
    if args.mode == "engine":
        qkv = [chart.GemvPlan(dev, [L["q"], L["k"], L["v"]], [ptr(x_attn)] * 3,
                              [ptr(outs["q"]), ptr(outs["k"]), ptr(outs["v"])]) for L in layers]
        gu = [chart.GemvPlan(dev, [L["gate"], L["up"]], [ptr(x_ffn)] * 2,
                             [ptr(outs["gate"]), ptr(outs["up"])]) for L in layers]
        plans = qkv + gu

        def layer_launch(i, s):
            L = layers[i]
            qkv[i].run(s)
            L["o"].gemv_f32_dev(ptr(xin["o"]), ptr(outs["o"]), s)
            gu[i].run(s)
            L["down"].gemv_f32_dev(ptr(xin["down"]), ptr(outs["down"]), s)

        n_windows = -(-n_sets // LAYERS)
        graphs = []
        cap = torch.cuda.Stream()
        for wdx in range(n_windows):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap):
                s = torch.cuda.current_stream().cuda_stream
                for l in range(LAYERS):
                    layer_launch((wdx * LAYERS + l) % n_sets, s)
            graphs.append(g)
        torch.cuda.synchronize()

        def step(i):
            graphs[i % n_windows].replay()
        launches_per_step = 4 * LAYERS
    else:
        n_windows = -(-n_sets // LAYERS)
        for wdx in range(n_windows):
            ws, xs, ys = [], [], []
            for l in range(LAYERS):
                L = layers[(wdx * LAYERS + l) % n_sets]
                for name, _, _ in SHAPES:
                    ws.append(L[name]), xs.append(ptr(xin[name])), ys.append(ptr(outs[name]))
            plans.append(chart.GemvPlan(dev, ws, xs, ys))

        def step(i):
            plans[i % n_windows].run(sh)
        launches_per_step = 1

    if args.only in (None, "gemv"):
        # Clock warm-up, untimed and before the W warm-up steps: an idle MI355X needs tens of ms of
        # load to reach its sustained clocks (20 steps ~ 1 ms left the timed region 15% slow), so
        # the hot path runs until CLOCK_WARMUP_S have passed.  Steady-state throughput is what a
        # busy serving GPU sees; the JSON line records the warm-up.
        t_w = time.perf_counter()
        n_clock = 0
        while time.perf_counter() - t_w < CLOCK_WARMUP_S:
            for _ in range(100):
                step(n_clock)
                n_clock += 1
            torch.cuda.synchronize()
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        assert dev.sync_status(sh) == 0
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        for i in range(args.steps):
            step(i)
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ev_ms = ev0.elapsed_time(ev1)
        ms_per_step = wall * 1e3 / args.steps
        value = step_bytes * args.steps / wall / 1e9
        log(f"[bench] config1 {args.mode}: {ms_per_step * 1e3:.1f} us/step, {value:.0f} GB/s wall, "
            f"{step_bytes * args.steps / (ev_ms / 1e3) / 1e9:.0f} GB/s events")

        # dominant kernel.  token: the plan launch, one per step, timed by the events over the timed
        # region.  engine: the per-layer launch with the most time, HIP events around each launch
        # on the launch stream (eager launches, rotating layers).
        kinds = {}
        if args.mode == "engine":
            kinds = {
                "qkv": (lambda i, s: qkv[i].run(s),
                        sum(proj_bytes(synth, t, n, k) for nm, n, k in SHAPES if nm in ("q", "k", "v"))),
                "o": (lambda i, s: layers[i]["o"].gemv_f32_dev(ptr(xin["o"]), ptr(outs["o"]), s),
                      proj_bytes(synth, t, 896, 896)),
                "gate_up": (lambda i, s: gu[i].run(s), 2 * proj_bytes(synth, t, 4864, 896)),
                "down": (lambda i, s: layers[i]["down"].gemv_f32_dev(ptr(xin["down"]), ptr(outs["down"]), s),
                         proj_bytes(synth, t, 896, 4864)),
            }
        per_kind = {}
        if args.mode == "token":
            # one launch per step: the timed region's events give the launch duration directly
            us = ev_ms * 1e3 / args.steps
            per_kind["token_plan"] = {"us": us, "bytes": step_bytes, "gbs": step_bytes / us / 1e3}
        reps = 64
        for name, (fn, nbytes) in kinds.items():
            evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in range(reps)]
            for i in range(8):
                fn(i % n_sets, sh)
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(evs):
                a.record(stream)
                fn((i * 7) % n_sets if args.mode == "engine" else i, sh)
                b.record(stream)
            torch.cuda.synchronize()
            us = float(np.mean([a.elapsed_time(b) for a, b in evs[4:]])) * 1e3
            per_kind[name] = {"us": us, "bytes": nbytes, "gbs": nbytes / us / 1e3}
        dom = max(per_kind, key=lambda k: per_kind[k]["us"])
        d = per_kind[dom]
        result["gemv"] = {
            "mode": args.mode, "launches_per_step": launches_per_step,
            "step_bytes": step_bytes, "ms_per_step": ms_per_step, "gbs_wall": value,
            "gbs_events": step_bytes * args.steps / (ev_ms / 1e3) / 1e9,
            "pool_gib": n_sets * layer_bytes_stored / 2**30,
            "kernels": per_kind,
        }
        result["_value"] = value
        result["_ms"] = ms_per_step
        traffic = measured_traffic() if args.mode == "token" else None
        result["roofline"] = {"bound": "hbm",
                              "kernel": ("gemv_stream_kernel<Q4_K> (token plan: 168 projections per launch)"
                                         if args.mode == "token" else f"gemv_stream_kernel<Q4_K> ({dom})"),
                              "achieved": round(d["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                              "frac": round(d["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                              "bytes_per_launch": d["bytes"], "us_per_launch": round(d["us"], 3)}

    for p in plans:
        p.free()

    # ---- config 3: N = 512 GEMMs ---------------------------------------------------------------
    if not args.no_gemm and args.only in (None, "gemm"):
        # The matrix-core ceiling measured on this device: MFMA-only loops on every CU.
        probe = {"int8_tops": round(dev.probe_mfma_peak(0), 1),
                 "f16_tflops": round(dev.probe_mfma_peak(1), 1)}
        log(f"[bench] MFMA-only probe: int8 32x32x32 {probe['int8_tops']:.0f} TOPS "
            f"({100 * probe['int8_tops'] / INT8_PEAK_TOPS:.1f}% of {INT8_PEAK_TOPS:.0f}), "
            f"f16 32x32x16 {probe['f16_tflops']:.0f} TFLOPS "
            f"({100 * probe['f16_tflops'] / F16_PEAK_TFLOPS:.1f}% of {F16_PEAK_TFLOPS:.0f})")
        result["mfma_probe"] = probe
        gemm = []
        n_tok = 512
        for gt in (synth.Q8_0, synth.Q4_K):
            for n_out, n_in in GEMM_SHAPES:
                rng = synth.rng_for(3, gt * 10 + n_in)
                raw = synth.payload(gt, rng, n_out, n_in)
                w = dev.upload(gt, raw, n_out, n_in)
                x = torch.from_numpy(synth.activations(rng, n_in, n_tok).reshape(n_tok, n_in)).cuda()
                codes = torch.empty((n_tok, n_in), dtype=torch.int8, device="cuda")
                scales = torch.empty((n_tok, -(-n_in // 32)), dtype=torch.int64, device="cuda")
                dev.quant_act_f32_dev(ptr(x), n_tok, n_in, ptr(codes), ptr(scales), sh)
                y = torch.empty((n_tok, n_out), dtype=torch.float32, device="cuda")
                t_w = time.perf_counter()  # clocks back up after the upload (untimed)
                while time.perf_counter() - t_w < 0.03:
                    for _ in range(5):
                        w.gemm_q8_dev(ptr(codes), ptr(scales), n_tok, ptr(y), sh)
                    torch.cuda.synchronize()
                assert dev.sync_status(sh) == 0
                reps = 50
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                for _ in range(reps):
                    w.gemm_q8_dev(ptr(codes), ptr(scales), n_tok, ptr(y), sh)
                b.record(stream)
                torch.cuda.synchronize()
                us = a.elapsed_time(b) * 1e3 / reps
                ops = 2.0 * n_tok * n_out * n_in
                tops = ops / us / 1e6
                wbytes = n_out * synth.needed_row_bytes(gt, n_in)
                traffic = wbytes + 4.0 * n_tok * n_out + n_tok * n_in  # weights + f32 out + int8 codes
                attain = min(INT8_PEAK_TOPS, ops / traffic * HBM_PEAK_GBS / 1e3)
                gemm.append({"type": synth.NAMES[gt], "shape": [n_out, n_in], "n_tok": n_tok,
                             "us": round(us, 2), "tops": round(tops, 1),
                             "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                             "frac_f16_probe": round(tops / probe["f16_tflops"], 4),
                             "attainable_tops": round(attain, 1),
                             "frac_attainable": round(tops / attain, 4)})
                log(f"[bench] gemm {synth.NAMES[gt]} {n_out}x{n_in} N{n_tok}: {us:.1f} us "
                    f"{tops:.0f} TOPS ({100 * tops / INT8_PEAK_TOPS:.1f}% int8 peak, "
                    f"{100 * tops / attain:.1f}% attainable)")
                w.free()
        result["gemm"] = gemm

    # ---- config 4: the 197 projections of a Qwen2.5-1.5B token (Q4_K + Q6_K), N = 1 and N = 512 ----
    # ---- configs[0] (Q8_0 4864x896) and configs[2] (151936x896 vocab head, Q6_K and Q8_0) ------
    # Single GEMV launches back to back over rotating weight copies of >= 1.1 GiB in all (the
    # 256 MB Infinity Cache cannot serve them), f32 N(0,1) input quantized in the kernel.
    if not args.no_heads and args.only in (None, "heads"):
        singles = []
        for cfg, gt, n_out, n_in in ((0, synth.Q8_0, 4864, 896), (2, synth.Q6_K, 151936, 896),
                                     (2, synth.Q8_0, 151936, 896)):
            raw = synth.payload(gt, synth.rng_for(cfg, gt), n_out, n_in)
            copies = max(2, -(-int(1.1 * 2 ** 30) // raw.nbytes))
            wc = [dev.upload(gt, raw, n_out, n_in) for _ in range(copies)]
            del raw
            x = torch.from_numpy(synth.activations(synth.rng_for(cfg, 99), n_in)).cuda()
            y = torch.empty(n_out, dtype=torch.float32, device="cuda")
            t_w = time.perf_counter()
            while time.perf_counter() - t_w < 0.05:  # clocks up after the uploads (untimed)
                for i in range(copies):
                    wc[i].gemv_f32_dev(ptr(x), ptr(y), sh)
                torch.cuda.synchronize()
            assert dev.sync_status(sh) == 0
            reps = 400 if n_out < 100000 else 60
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for i in range(reps):
                wc[i % copies].gemv_f32_dev(ptr(x), ptr(y), sh)
            b.record(stream)
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1e3 / reps
            nbytes = proj_bytes(synth, gt, n_out, n_in)
            gbs = nbytes / us / 1e3
            singles.append({"config": cfg, "type": synth.NAMES[gt], "shape": [n_out, n_in],
                            "copies": copies, "us": round(us, 2), "bytes": nbytes,
                            "gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
            log(f"[bench] config{cfg} {synth.NAMES[gt]} {n_out}x{n_in}: {us:.2f} us/launch, {gbs:.0f} GB/s "
                f"= {100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s ({copies} rotating copies)")
            for w in wc:
                w.free()
            del wc
        result["heads"] = singles

    if not args.no_config4 and args.only in (None, "config4"):
        projs = cfg4_projections(synth)
        host = {}
        for (gt, n_out, n_in) in set(projs):
            host[(gt, n_out, n_in)] = synth.payload(gt, synth.rng_for(4, gt * 100000 + n_out + n_in), n_out, n_in)
        ws = [dev.upload(gt, host[(gt, n_out, n_in)], n_out, n_in) for gt, n_out, n_in in projs]
        del host
        tok_bytes = sum(proj_bytes(synth, gt, n_out, n_in) for gt, n_out, n_in in projs)
        rng = synth.rng_for(4, 1)
        x1 = {k: torch.from_numpy(synth.activations(rng, k)).cuda() for k in (1536, 8960)}
        y1 = {}
        for gt, n_out, n_in in projs:
            y1.setdefault(n_out, torch.zeros(n_out, dtype=torch.float32, device="cuda"))
        # N = 1: the token's 197 projections as one launch per quant type (the projections of a
        # token are independent here, as in configs[1]), and for comparison as one mixed-type
        # launch; the 0.98 GB of weights per token is past the 256 MB Infinity Cache
        mixed = [chart.GemvPlan(dev, ws, [ptr(x1[p[2]]) for p in projs], [ptr(y1[p[1]]) for p in projs])]
        by_type = []
        for gt in (synth.Q4_K, synth.Q6_K):
            idx = [i for i, p in enumerate(projs) if p[0] == gt]
            by_type.append(chart.GemvPlan(dev, [ws[i] for i in idx], [ptr(x1[projs[i][2]]) for i in idx],
                                          [ptr(y1[projs[i][1]]) for i in idx]))

        def tok_us(plans, reps=20):
            for _ in range(3):
                for p in plans:
                    p.run(sh)
            torch.cuda.synchronize()
            assert dev.sync_status(sh) == 0
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(reps):
                for p in plans:
                    p.run(sh)
            b.record(stream)
            torch.cuda.synchronize()
            return a.elapsed_time(b) * 1e3 / reps
        tok_us(by_type)  # clocks up
        us_mixed = min(tok_us(mixed), tok_us(mixed))
        us_tok = min(tok_us(by_type), tok_us(by_type))
        gbs = tok_bytes / us_tok / 1e3
        log(f"[bench] config4 N=1: {us_tok:.1f} us/token ({len(projs)} projections, one launch per type), "
            f"{gbs:.0f} GB/s = {100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s; one mixed-type launch: {us_mixed:.1f} us")
        for p in mixed + by_type:
            p.free()
        # N = 512: one GEMM per projection, f32 inputs quantized in the operand pass
        n_tok = 512
        xs = {k: torch.from_numpy(synth.activations(rng, k, n_tok).reshape(n_tok, k)).cuda() for k in (1536, 8960)}
        ys = {}
        for gt, n_out, n_in in projs:
            ys.setdefault(n_out, torch.empty((n_tok, n_out), dtype=torch.float32, device="cuda"))

        # one grouped call per shared input, as a layer feeds them: q/k/v (the attention input),
        # o, gate/up (the FFN input), down; the head alone.  7 projections -> 4 operand passes.
        groups, i = [], 0
        while i < len(projs):
            n = 3 if i % 7 == 0 and i + 3 <= len(projs) - 1 else 2 if i % 7 == 4 else 1
            groups.append(list(range(i, i + n)))
            i += n

        def prefill():
            for g in groups:
                n_in = projs[g[0]][2]
                chart.gemm_group_f32_dev(dev, [ws[j] for j in g], ptr(xs[n_in]), n_tok,
                                         [ptr(ys[projs[j][1]]) for j in g], sh)
        prefill()
        torch.cuda.synchronize()
        assert dev.sync_status(sh) == 0
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(2):
            prefill()
        b.record(stream)
        torch.cuda.synchronize()
        ms_pre = a.elapsed_time(b) / 2
        ops = sum(2.0 * n_tok * n_out * n_in for _, n_out, n_in in projs)
        tops = ops / ms_pre / 1e9
        log(f"[bench] config4 N=512: {ms_pre:.2f} ms/prefill ({len(projs)} GEMMs in {len(groups)} grouped "
            f"calls, one operand pass each), {tops:.0f} TOPS = "
            f"{100 * tops / INT8_PEAK_TOPS:.1f}% int8 peak")
        result["config4"] = {"projections": len(projs), "n1_us_per_token": round(us_tok, 1),
                             "n1_bytes_per_token": tok_bytes, "n1_gbs": round(gbs, 1),
                             "n1_frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "n1_launches": 2,
                             "n1_us_one_mixed_launch": round(us_mixed, 1),
                             "n512_ms": round(ms_pre, 3), "n512_tops": round(tops, 1),
                             "n512_grouped_calls": len(groups),
                             "n512_frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        for w in ws:
            w.free()
        del xs, ys, x1, y1

    # ---- CPU baseline: the same config-1 step on the host (restated reference fast path) ----------
    if not args.no_cpu and args.only in (None, "gemv"):
        import oracle

        threads = max(1, min(args.cpu_threads, os.cpu_count() or 1))
        xq = {}
        for name, _, k in SHAPES:
            xq[name] = xin[name].cpu().numpy()

        def cpu_step(li):
            src = host_layers[li % n_unique]
            st, c_attn, s_attn = oracle.quant_act_f32(xq["q"])
            for name in ("q", "k", "v"):
                n, k = next((n, k) for nm, n, k in SHAPES if nm == name)
                oracle.matvec_q8act_fast(t, src[name], n, k, c_attn, s_attn, threads)
            st, c, s = oracle.quant_act_f32(xq["o"])
            oracle.matvec_q8act_fast(t, src["o"], 896, 896, c, s, threads)
            st, c, s = oracle.quant_act_f32(xq["gate"])
            oracle.matvec_q8act_fast(t, src["gate"], 4864, 896, c, s, threads)
            oracle.matvec_q8act_fast(t, src["up"], 4864, 896, c, s, threads)
            st, c, s = oracle.quant_act_f32(xq["down"])
            oracle.matvec_q8act_fast(t, src["down"], 896, 4864, c, s, threads)

        # host pool: distinct copies past the host LLC, like the GPU pool
        host_pool = [{nm: host_layers[i % n_unique][nm].copy() for nm, _, _ in SHAPES}
                     for i in range(48)]
        host_layers = host_pool
        n_unique = len(host_pool)
        cpu_step(0)
        layers_done = 0
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds:
            cpu_step(layers_done)
            layers_done += 1
        el = time.perf_counter() - t0
        layer_bytes = step_bytes / LAYERS
        cpu_gbs = layers_done * layer_bytes / el / 1e9
        result["cpu_baseline"] = {
            "value": round(cpu_gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{layers_done} layers ({layers_done / LAYERS:.1f} config-1 steps) of the 7 Q4_K "
                      f"projections, f32 input quantized per call, {el:.1f} s on {threads} threads, "
                      f"48 rotating layer copies ({48 * layer_bytes_stored / 2**30:.2f} GiB)",
            "cpu": _cpu_name(), "host_cpus": os.cpu_count(),
        }
        log(f"[bench] cpu baseline: {cpu_gbs:.1f} GB/s on {threads} threads")

    if args.only not in (None, "gemv"):
        print(json.dumps(result))
        return 0

    line = {
        "metric": "quant GEMV HBM GB/s (N=1) + int8-MFMA GEMM TOPS (N=512), % of roofline",
        "value": round(result["_value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_warmup_ms": round(CLOCK_WARMUP_S * 1e3),
        "ms_per_step": round(result["_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xQ4_K (exact int32 group dots, f32 fold)",
        "data": "synthetic (BASELINE.json configs[1] distributions, seeded)",
        "config": {"workload": "configs[1]: Q4_K GEMV decode N=1, Qwen2.5-0.5B projections "
                               "(q,k,v,o,gate,up,down) x 24 layers per step, weights rotated "
                               f"through a {result['gemv']['pool_gib']:.2f} GiB pool",
                   "mode": args.mode, "parallelism": "single GPU"},
        "roofline": result["roofline"],
        "cpu_baseline": result.get("cpu_baseline"),
        "gemv": result["gemv"],
        "gemm": result.get("gemm"),
        "mfma_probe": result.get("mfma_probe"),
        "config4": result.get("config4"),
        "config0_config2": result.get("heads"),
    }
    print(json.dumps(line))
    dev.close()
    return 0


def _cpu_name() -> str:
    try:
        for l in open("/proc/cpuinfo"):
            if l.startswith("model name"):
                return l.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
