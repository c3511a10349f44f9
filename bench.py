#!/usr/bin/env python3
"""Benchmark of the quantized linear-layer path on one MI355X.

Headline (the largest single-GPU configuration): one decode token (N = 1)
through every linear layer of a random-init Qwen2.5-1.5B-architecture model in the Q4_K_M-style mix
(hidden 1536, 28 layers, KV width 256, FFN 8960, vocab 151936; Q4_K everywhere except Q6_K for
attn_v, ffn_down on llama.cpp's use_more_bits layers and the output head).  One step is one token,
run as a dependency-respecting sequence: per layer q/k/v (one grouped launch: they share their
input) -> o -> gate/up (one grouped launch) -> down, then the head -- 113 dependent stage launches,
each waiting for the previous one (stream order), replayed as one HIP graph per token.  The engine's
own operations between stages (attention, RMSNorm, SwiGLU, residuals) are not on this path; each
stage reads its own HBM-resident f32 input.  The 0.99 GB of weights per token is past the 256 MB
Infinity Cache, so every token streams its weights from HBM.

value = algorithmic bytes per token * steps / wall time (GB/s).  Algorithmic bytes per projection
= n_out * (weight bytes a correct kernel must read per row) + 4*n_in (f32 input) + 4*n_out (f32
output).

Timing: the hot path first runs untimed for 150 ms (clock ramp-up of an idle GPU), then the W
warm-up steps, then the K timed steps between two synchronizations.

Also reported, beside the value:
  roofline      the token's dominant kernel (the Q4_K stage launches, o / gate-up / Q4_K down:
                most of a token's time) against the 8 TB/s HBM peak, HIP events on the launch
                stream around replays of one graph of those launches in token order;
  decode        the same token as eager launches; with the fused FFN in launch form (gate/up with
                the exact SwiGLU + hidden requantize in one launch, down from the hidden codes:
                the FFN's real data dependency) and, its baseline, with the plain gate/up launch
                then the SwiGLU as a launch of its own; as one persistent launch (ah_seq_*, with and
                without the fused FFN's SwiGLU stage); with its 197 projections batched as
                independent parts (two launches: not a dependency-respecting token); and the
                launch floor: a graph of 113 minimal launches on one stream;
  config1       BASELINE configs[1] (Qwen2.5-0.5B, 24 layers, Q4_K) as one batched launch;
  gemm          configs[3] N = 512 GEMMs against the 5.0 POPS int8 MFMA peak (Q8_0 on both MFMA
                designs, int8 and f16; Q4_K on the f16, the dequantize-once tile and the int8
                designs), each from pre-quantized codes and from the f32 input, the MFMA-only probe, the configs[4]
                N = 512 prefill, and its FFN fused (gate/up + exact SwiGLU + hidden quant_act in one
                launch) and two-pass (--only gemm3: the configs[3] GEMMs alone, for profiling);
  heads         configs[0] (Q8_0 4864x896) and configs[2] (151936x896 head, Q6_K and Q8_0);
  families      Q5_0, Q2_K and Q3_K: a 151936x896 launch (bandwidth), a 4864x896 launch
                (latency) and the N = 512 GEMM at 4864x896 (Q2_K / Q3_K on the dequantize-once
                tiles, and on the per-token GEMV route for comparison);
  cpu_baseline  the restated reference fast path (oracle/ah_cpu_fast.c: AVX-VNNI or AVX2 dots,
                two-row tiles) on the same token's projections, on this host's cores;
                cpu_baseline_gemm the same for all 512 columns of the four configs[3] shapes per
                type, at --cpu-threads and at all host cores.
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
# Qwen2.5-0.5B projections
CFG1_LAYERS = 24
CFG1_SHAPES = [("q", 896, 896), ("k", 128, 896), ("v", 128, 896), ("o", 896, 896),
               ("gate", 4864, 896), ("up", 4864, 896), ("down", 896, 4864)]
GEMM_SHAPES = [(4864, 896), (896, 4864), (8960, 1536), (1536, 8960)]
# Qwen2.5-1.5B architecture, Q4_K_M-style mix (Q6_K for attn_v, for ffn_down on
# llama.cpp's use_more_bits layers, and for the output head)
CFG4_LAYERS = 28
CFG4_Q6K_DOWN = {0, 1, 2, 5, 8, 11, 14, 17, 20, 23, 24, 25, 26, 27}
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode_config4_token.md")


def cfg4_layer(synth, l):
    """configs[4] layer l: (name, ggml type, n_out, n_in) in the engine's projection order."""
    return [("q", synth.Q4_K, 1536, 1536), ("k", synth.Q4_K, 256, 1536), ("v", synth.Q6_K, 256, 1536),
            ("o", synth.Q4_K, 1536, 1536), ("gate", synth.Q4_K, 8960, 1536), ("up", synth.Q4_K, 8960, 1536),
            ("down", synth.Q6_K if l in CFG4_Q6K_DOWN else synth.Q4_K, 1536, 8960)]


CFG4_STAGES = [("qkv", ("q", "k", "v")), ("o", ("o",)), ("gate_up", ("gate", "up")), ("down", ("down",))]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def proj_bytes(synth, t, n_out, n_in):
    return n_out * synth.needed_row_bytes(t, n_in) + 4 * n_in + 4 * n_out


def profile_value(key, cast=float):
    """A figure of the roofline kernel from the committed rocprofv3 summary: the HBM bytes per
    launch from its FETCH_SIZE / WRITE_SIZE runs (copy-calibrated; the counters cannot be read from
    inside this process) or its kernel-only average duration; None when not committed."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return cast(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_flags():
    try:
        for l in open("/proc/cpuinfo"):
            if l.startswith("flags"):
                f = set(l.split(":", 1)[1].split())
                return {"avx2": "avx2" in f, "avx_vnni": "avx_vnni" in f, "avx512f": "avx512f" in f,
                        "avx512_vnni": "avx512_vnni" in f}
    except OSError:
        pass
    return {}


def _cpu_name() -> str:
    try:
        for l in open("/proc/cpuinfo"):
            if l.startswith("model name"):
                return l.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-heads", action="store_true", help="skip configs[0] and configs[2]")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="headline only (decode token + roofline)")
    ap.add_argument("--cpu-seconds", type=float, default=6.0)
    ap.add_argument("--cpu-threads", type=int, default=8)
    ap.add_argument("--no-seq", action="store_true",
                    help="skip the persistent (one-launch) token forms of the decode extras")
    ap.add_argument("--only", choices=["decode", "gemm", "gemm3", "config1", "heads", "families", "copy"],
                    default=None)
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
    result: dict = {}

    def ptr(x):
        return x.data_ptr()

    if args.only == "copy":
        # calibration for the FETCH_SIZE / WRITE_SIZE counters: a plain 256 MiB copy
        a = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": a.numel()}))
        return 0

    def clock_up(fn, seconds=CLOCK_WARMUP_S):
        t_w = time.perf_counter()
        while time.perf_counter() - t_w < seconds:
            for _ in range(10):
                fn()
            torch.cuda.synchronize()

    def event_us(fn, reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) * 1e3 / reps

    # ---- weights (one device copy per projection, 0.99 GB) --------------------------
    run_decode = args.only in (None, "decode")
    run_prefill = args.only in (None, "gemm") and not args.no_gemm and not args.no_extras
    if run_decode or run_prefill:
        host = {}
        spec = [cfg4_layer(synth, l) for l in range(CFG4_LAYERS)]
        for layer in spec:
            for _, gt, n_out, n_in in layer:
                if (gt, n_out, n_in) not in host:
                    host[(gt, n_out, n_in)] = synth.payload(gt, synth.rng_for(4, gt * 100000 + n_out + n_in), n_out, n_in)
        head_key = (synth.Q6_K, 151936, 1536)
        host[head_key] = synth.payload(synth.Q6_K, synth.rng_for(4, 7), 151936, 1536)
        W = [{nm: (gt, n_out, n_in, dev.upload(gt, host[(gt, n_out, n_in)], n_out, n_in))
              for nm, gt, n_out, n_in in layer} for layer in spec]
        head = dev.upload(synth.Q6_K, host[head_key], 151936, 1536)
        tok_bytes = sum(proj_bytes(synth, gt, n_out, n_in) for layer in spec for _, gt, n_out, n_in in layer)
        tok_bytes += proj_bytes(synth, *head_key)
        rng = synth.rng_for(4, 1)
        X = {nm: torch.from_numpy(synth.activations(rng, k)).cuda()
             for nm, k in (("attn", 1536), ("o", 1536), ("ffn", 1536), ("down", 8960), ("head", 1536))}
        Y = {nm: torch.zeros(n, dtype=torch.float32, device="cuda")
             for nm, n in (("q", 1536), ("k", 256), ("v", 256), ("o", 1536), ("gate", 8960), ("up", 8960),
                           ("down", 1536), ("head", 151936))}
        src = {"q": "attn", "k": "attn", "v": "attn", "o": "o", "gate": "ffn", "up": "ffn", "down": "down"}

    if run_decode:
        # the token's 113 dependent stages, one plan (one launch) each
        plans, kinds = [], []
        for L in W:
            for kind, names in CFG4_STAGES:
                plans.append(chart.GemvPlan(dev, [L[n][3] for n in names], [ptr(X[src[n]]) for n in names],
                                            [ptr(Y[n]) for n in names]))
                kinds.append((kind, sum(proj_bytes(synth, *L[n][:3]) for n in names),
                              tuple(sorted({L[n][0] for n in names}))))
        plans.append(chart.GemvPlan(dev, [head], [ptr(X["head"])], [ptr(Y["head"])]))
        kinds.append(("head", proj_bytes(synth, *head_key), (synth.Q6_K,)))

        def token_eager():
            for p in plans:
                p.run(sh)

        token_eager()
        torch.cuda.synchronize()
        assert dev.sync_status(sh) == 0
        graph = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream()
        with torch.cuda.graph(graph, stream=cap):
            s_cap = torch.cuda.current_stream().cuda_stream
            for p in plans:
                p.run(s_cap)
        torch.cuda.synchronize()
        step = graph.replay

        clock_up(step)
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        assert dev.sync_status(sh) == 0
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        ev0.record(stream)
        for _ in range(args.steps):
            step()
        ev1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ev_ms = ev0.elapsed_time(ev1)
        assert dev.sync_status(sh) == 0
        ms_per_step = wall * 1e3 / args.steps
        value = tok_bytes * args.steps / wall / 1e9
        log(f"[bench] configs[4] decode token (graph of {len(plans)} dependent stage launches): "
            f"{ms_per_step * 1e3:.1f} us/token, {value:.0f} GB/s wall, "
            f"{tok_bytes * args.steps / (ev_ms / 1e3) / 1e9:.0f} GB/s events")

        # Per stage kind: the kind's launches back to back in token order (eager, HIP events on the
        # launch stream over 4 passes).  The roofline kernel is gemv_stream_kernel<Q4_K> (plan form):
        # the o, gate/up and Q4_K down launches, which take most of a token.
        per_kind = {}
        for kind in ("qkv", "o", "gate_up", "down", "head"):
            idx = [i for i, k in enumerate(kinds) if k[0] == kind]
            reps = 4 if kind != "head" else 40
            us = event_us(lambda: [plans[i].run(sh) for i in idx], reps) / len(idx)
            nbytes = sum(kinds[i][1] for i in idx) / len(idx)
            per_kind[kind] = {"launches_per_token": len(idx), "us_per_launch": round(us, 2),
                              "bytes_per_launch": int(nbytes), "gbs": round(nbytes / us / 1e3, 1),
                              "us_per_token": round(us * len(idx), 1)}
        # The roofline kernel's launches, timed as the token runs them: the Q4_K stage launches in
        # token order captured into one graph, replayed on the launch stream between HIP events.
        q4 = [i for i, k in enumerate(kinds) if k[2] == (synth.Q4_K,)]
        graph_q4 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph_q4, stream=cap):
            s_q4 = torch.cuda.current_stream().cuda_stream
            for i in q4:
                plans[i].run(s_q4)
        torch.cuda.synchronize()
        clock_up(graph_q4.replay, 0.05)
        us_q4 = min(event_us(graph_q4.replay, 10) for _ in range(3)) / len(q4)
        us_q4_eager = event_us(lambda: [plans[i].run(sh) for i in q4], 4) / len(q4)
        b_q4 = sum(kinds[i][1] for i in q4) / len(q4)
        assert dev.sync_status(sh) == 0
        del graph_q4
        traffic = profile_value("traffic_bytes_per_launch", int)
        result["roofline"] = {
            "bound": "hbm",
            "kernel": f"gemv_stream_kernel<Q4_K> plan launches of the token ({len(q4)} per token: "
                      "o, gate/up and the Q4_K down projections)",
            "achieved": round(b_q4 / us_q4 / 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(b_q4 / us_q4 / 1e3 / HBM_PEAK_GBS, 4), "traffic": traffic,
            "bytes_per_launch": int(b_q4), "us_per_launch": round(us_q4, 3),
            "us_per_launch_eager": round(us_q4_eager, 3),
            "note": "us_per_launch: HIP events around replays of one graph of these launches in token "
                    "order (the dependent chain as the token runs it); us_per_launch_eager: the same "
                    "launches back to back from the host; traffic and kernel_us_profile: the committed "
                    "rocprofv3 summary (profiles/decode_config4_token.md)",
            "kernel_us_profile": profile_value("kernel_us_per_launch")}
        result["_value"], result["_ms"] = value, ms_per_step
        decode = {"stages": len(plans), "bytes_per_token": tok_bytes, "us_per_token_graph": round(ms_per_step * 1e3, 1),
                  "gbs_graph": round(value, 1), "gbs_events": round(tok_bytes * args.steps / (ev_ms / 1e3) / 1e9, 1),
                  "per_stage_kind": per_kind}

        if not args.no_extras:
            reps = 20
            decode["us_per_token_eager"] = round(event_us(token_eager, reps), 1)
            # the token with the fused FFN in launch form (ffn_q8act_prepared_into): per layer q/k/v
            # -> o -> gate/up with the exact SwiGLU and hidden requantize in one launch
            # (ah_ffn_gate_up_dev) -> down from the hidden codes, then the head: 85 launches, one graph
            hc_g = torch.zeros(8960, dtype=torch.int8, device="cuda")
            hs_g = torch.zeros(280, dtype=torch.int64, device="cuda")

            def token_fused(s):
                for li, L in enumerate(W):
                    plans[4 * li].run(s)
                    plans[4 * li + 1].run(s)
                    chart.ffn_dev(dev, L["gate"][3], L["up"][3], L["down"][3], ptr(X["ffn"]), ptr(Y["down"]),
                                  ptr(hc_g), ptr(hs_g), s)
                plans[-1].run(s)

            graph_f = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph_f, stream=cap):
                token_fused(torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            clock_up(graph_f.replay, 0.05)
            decode["us_per_token_graph_fused_ffn"] = round(event_us(graph_f.replay, reps), 1)
            assert dev.sync_status(sh) == 0
            del graph_f
            # its like-for-like baseline: the plain gate/up launch, then the SwiGLU + hidden quantizer
            # as a launch of its own (ah_swiglu_quant_dev), then down from the hidden codes
            def token_swiglu(s):
                for li, L in enumerate(W):
                    plans[4 * li].run(s)
                    plans[4 * li + 1].run(s)
                    plans[4 * li + 2].run(s)
                    chart.swiglu_quant_dev(dev, ptr(Y["gate"]), ptr(Y["up"]), 1, 8960, ptr(hc_g), ptr(hs_g), s)
                    L["down"][3].gemv_q8_dev(ptr(hc_g), ptr(hs_g), ptr(Y["down"]), s)
                plans[-1].run(s)

            graph_s = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph_s, stream=cap):
                token_swiglu(torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            clock_up(graph_s.replay, 0.05)
            decode["us_per_token_graph_plain_then_swiglu"] = round(event_us(graph_s.replay, reps), 1)
            assert dev.sync_status(sh) == 0
            del graph_s
            # the launch floor of a dependent token: a graph of as many minimal launches (a one-element
            # fill each) on one stream as the token has stages
            tiny = torch.zeros(1, dtype=torch.float32, device="cuda")
            graph_e = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph_e, stream=cap):
                for _ in range(len(plans)):
                    tiny.fill_(1.0)
            torch.cuda.synchronize()
            clock_up(graph_e.replay, 0.05)
            decode["floor_us_per_token"] = round(event_us(graph_e.replay, reps), 1)
            decode["floor_launches"] = len(plans)
            del graph_e
            # one persistent launch per token (ah_seq_*): the same stages; and with the fused FFN's
            # SwiGLU stage between gate/up and down (down then reads the hidden QuantAct)
            hc = torch.zeros(8960, dtype=torch.int8, device="cuda")
            hs = torch.zeros(280, dtype=torch.int64, device="cuda")
            for fused in (() if args.no_seq else (False, True)):
                stages = []
                for L in W:
                    part = lambda n, x=None: (L[n][3], x if x is not None else ptr(X[src[n]]), ptr(Y[n]))
                    stages += [("gemv", [part("q"), part("k"), part("v")]), ("gemv", [part("o")]),
                               ("gemv", [part("gate"), part("up")])]
                    if fused:
                        stages += [("swiglu", ptr(Y["gate"]), ptr(Y["up"]), 8960, ptr(hc), ptr(hs)),
                                   ("gemv", [part("down", (ptr(hc), ptr(hs)))])]
                    else:
                        stages += [("gemv", [part("down")])]
                stages.append(("gemv", [(head, ptr(X["head"]), ptr(Y["head"]))]))
                seq = chart.Seq(dev, stages)
                clock_up(lambda: seq.run(sh), 0.05)
                us = event_us(lambda: seq.run(sh), reps)
                st = seq.sync_status(sh)
                assert st == (0, 0), st
                decode["us_per_token_persistent" + ("_fused_ffn" if fused else "")] = round(us, 1)
                seq.free()
            # the 197 projections batched as independent parts, one launch per quant type (not a
            # dependency-respecting token: the rate of the streaming kernel alone)
            flat = [(L[n], n) for L in W for n in ("q", "k", "v", "o", "gate", "up", "down")]
            by_type = []
            for gt in (synth.Q4_K, synth.Q6_K):
                sel = [(w, n) for w, n in flat if w[0] == gt]
                ws = [w[3] for w, _ in sel] + ([head] if gt == synth.Q6_K else [])
                xs = [ptr(X[src[n]]) for _, n in sel] + ([ptr(X["head"])] if gt == synth.Q6_K else [])
                ys = [ptr(Y[n]) for _, n in sel] + ([ptr(Y["head"])] if gt == synth.Q6_K else [])
                by_type.append(chart.GemvPlan(dev, ws, xs, ys))
            clock_up(lambda: [p.run(sh) for p in by_type], 0.05)
            us_b = event_us(lambda: [p.run(sh) for p in by_type], reps)
            decode["us_per_token_independent_parts"] = round(us_b, 1)
            decode["gbs_independent_parts"] = round(tok_bytes / us_b / 1e3, 1)
            for p in by_type:
                p.free()
            assert dev.sync_status(sh) == 0
            log(f"[bench] decode token: eager {decode['us_per_token_eager']} us, graph with the fused FFN "
                f"{decode['us_per_token_graph_fused_ffn']} us, persistent "
                f"{decode.get('us_per_token_persistent')} us, persistent with fused FFN "
                f"{decode.get('us_per_token_persistent_fused_ffn')} us, independent parts {us_b:.1f} us")
        result["decode"] = decode
        for p in plans:
            p.free()

    # ---- configs[4] prefill, N = 512: grouped GEMMs as a layer feeds them -------------------------
    if run_prefill:
        n_tok = 512
        xs = {k: torch.from_numpy(synth.activations(rng, k, n_tok).reshape(n_tok, k)).cuda() for k in (1536, 8960)}
        ys = {nm: torch.empty((n_tok, n), dtype=torch.float32, device="cuda")
              for nm, n in (("q", 1536), ("k", 256), ("v", 256), ("o", 1536), ("gate", 8960), ("up", 8960),
                            ("down", 1536), ("head", 151936))}
        groups = []
        for L in W:
            for _, names in CFG4_STAGES:
                groups.append(([L[n][3] for n in names], names[0] == "down", list(names)))
        groups.append(([head], False, ["head"]))

        def prefill():
            for ws, is_down, outs in groups:
                chart.gemm_group_f32_dev(dev, ws, ptr(xs[8960 if is_down else 1536]), n_tok,
                                         [ptr(ys[n]) for n in outs], sh)
        prefill()
        torch.cuda.synchronize()
        assert dev.sync_status(sh) == 0
        ms_pre = event_us(prefill, 2) / 1e3
        ops = sum(2.0 * n_tok * w[1] * w[2] for L in W for w in L.values()) + 2.0 * n_tok * 151936 * 1536
        tops = ops / ms_pre / 1e9
        log(f"[bench] configs[4] N=512 prefill: {ms_pre:.2f} ms ({len(groups)} grouped calls), {tops:.0f} TOPS "
            f"= {100 * tops / INT8_PEAK_TOPS:.1f}% int8 peak")
        result["config4_prefill"] = {"n_tok": n_tok, "ms": round(ms_pre, 3), "tops": round(tops, 1),
                                     "grouped_calls": len(groups), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        del xs, ys
    if run_decode or run_prefill:
        for L in W:
            for w in L.values():
                w[3].free()
        head.free()

    # ---- N = 512 GEMMs ------------------------------------------------------------------
    if args.only in (None, "gemm", "gemm3") and not args.no_gemm and not args.no_extras:
        if args.only == "gemm3":
            probe = {"int8_tops": INT8_PEAK_TOPS, "f16_tflops": INT8_PEAK_TOPS / 2}  # published peaks
        else:
            probe = {"int8_tops": round(dev.probe_mfma_peak(0), 1), "f16_tflops": round(dev.probe_mfma_peak(1), 1)}
            log(f"[bench] MFMA-only probe: int8 32x32x32 {probe['int8_tops']:.0f} TOPS, "
                f"f16 32x32x16 {probe['f16_tflops']:.0f} TFLOPS")
            result["mfma_probe"] = probe
        gemm = []
        n_tok = 512
        # Q8_0 on both MFMA designs (int8, the default, and f16); Q4_K on the f16 design (the
        # default), the dequantize-once tiles and the int8 design
        for gt, design in ((synth.Q8_0, chart.Device.GEMM_INT8), (synth.Q8_0, chart.Device.GEMM_F16),
                           (synth.Q4_K, chart.Device.GEMM_F16), (synth.Q4_K, chart.Device.GEMM_F16_TILE),
                           (synth.Q4_K, chart.Device.GEMM_INT8)):
            dname = {chart.Device.GEMM_INT8: "int8", chart.Device.GEMM_F16: "f16",
                     chart.Device.GEMM_F16_TILE: "f16 tiles"}[design]
            dev.set_gemm_design(gt, design)
            for n_out, n_in in GEMM_SHAPES:
                rng3 = synth.rng_for(3, gt * 10 + n_in)
                w = dev.upload(gt, synth.payload(gt, rng3, n_out, n_in), n_out, n_in)
                x = torch.from_numpy(synth.activations(rng3, n_in, n_tok).reshape(n_tok, n_in)).cuda()
                codes = torch.empty((n_tok, n_in), dtype=torch.int8, device="cuda")
                scales = torch.empty((n_tok, -(-n_in // 32)), dtype=torch.int64, device="cuda")
                dev.quant_act_f32_dev(ptr(x), n_tok, n_in, ptr(codes), ptr(scales), sh)
                y = torch.empty((n_tok, n_out), dtype=torch.float32, device="cuda")
                run = lambda: w.gemm_q8_dev(ptr(codes), ptr(scales), n_tok, ptr(y), sh)
                clock_up(run, 0.03)
                assert dev.sync_status(sh) == 0
                us = event_us(run, 50)
                # the same GEMM from the f32 input (the quantizer pass inside the timing, as configs[3]
                # specifies it)
                run_f = lambda: w.gemm_f32_dev(ptr(x), n_tok, ptr(y), sh)
                clock_up(run_f, 0.02)
                assert dev.sync_status(sh) == 0
                us_f = event_us(run_f, 50)
                ops = 2.0 * n_tok * n_out * n_in
                tops = ops / us / 1e6
                traffic = n_out * synth.needed_row_bytes(gt, n_in) + 4.0 * n_tok * n_out + n_tok * n_in
                attain = min(INT8_PEAK_TOPS, ops / traffic * HBM_PEAK_GBS / 1e3)
                gemm.append({"type": synth.NAMES[gt], "design": dname, "shape": [n_out, n_in], "n_tok": n_tok,
                             "us": round(us, 2), "tops": round(tops, 1),
                             "us_f32_input": round(us_f, 2), "tops_f32_input": round(ops / us_f / 1e6, 1),
                             "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                             "frac_f16_probe": round(tops / probe["f16_tflops"], 4),
                             "attainable_tops": round(attain, 1), "frac_attainable": round(tops / attain, 4)})
                log(f"[bench] gemm {synth.NAMES[gt]} ({dname} MFMA) {n_out}x{n_in} N{n_tok}: {us:.1f} us "
                    f"{tops:.0f} TOPS ({100 * tops / INT8_PEAK_TOPS:.1f}% int8 peak); from f32 {us_f:.1f} us")
                w.free()
            dev.set_gemm_design(gt, chart.Device.GEMM_AUTO)
        result["gemm"] = gemm

        # configs[4] prefill FFN at N = 512 (gate/up Q4_K 8960x1536, down Q6_K 1536x8960): the fused
        # gate/up launch (SwiGLU + hidden quant_act in the tiles' epilogue) against the two-pass
        # form (grouped gate/up GEMM, then the SwiGLU pass), alone and with the down projection
        # (gate/up rows centred on zero, as trained FFN weights are: q4_k_payload's common positive
        # row bias makes ~1 token in 16 a hidden vector the f16 band cannot carry, which the down
        # GEMM then serves on its exact path -- measured below as down_exact_path)
        rngf = synth.rng_for(4, 77)
        Gf = dev.upload(synth.Q4_K, synth.q4_k_centered_payload(rngf, 8960, 1536), 8960, 1536)
        Uf = dev.upload(synth.Q4_K, synth.q4_k_centered_payload(rngf, 8960, 1536), 8960, 1536)
        Df = dev.upload(synth.Q6_K, synth.payload(synth.Q6_K, rngf, 1536, 8960), 1536, 8960)
        xf = torch.from_numpy(synth.activations(rngf, 1536, n_tok).reshape(n_tok, 1536).astype(np.float32)).cuda()
        hcf = torch.empty((n_tok, 8960), dtype=torch.int8, device="cuda")
        hsf = torch.empty((n_tok, 280), dtype=torch.int64, device="cuda")
        yf = torch.empty((n_tok, 1536), dtype=torch.float32, device="cuda")
        ffn = {"n_tok": n_tok, "shapes": {"gate_up": [8960, 1536], "down": [1536, 8960]},
               "types": {"gate_up": "Q4_K", "down": "Q6_K"}}
        gu_ops = 2 * 2.0 * n_tok * 8960 * 1536
        for fused in (True, False):
            dev.set_ffn_prefill_form(chart.Device.FFN_FUSED if fused else chart.Device.FFN_TWO_PASS)
            gu = lambda: chart.ffn_gate_up_prefill_dev(dev, Gf, Uf, ptr(xf), n_tok, ptr(hcf), ptr(hsf), None, None, sh)
            whole = lambda: chart.ffn_prefill_dev(dev, Gf, Uf, Df, ptr(xf), n_tok, ptr(yf), ptr(hcf), ptr(hsf), sh)
            clock_up(gu, 0.03)
            assert dev.sync_status(sh) == 0, "ffn prefill refused (synthetic scale)"
            key = "fused" if fused else "two_pass"
            us_gu = event_us(gu, 20)
            clock_up(whole, 0.02)
            assert dev.sync_status(sh) == 0
            us_all = event_us(whole, 20)
            ffn[key] = {"gate_up_us": round(us_gu, 2), "gate_up_tops": round(gu_ops / us_gu / 1e6, 1),
                        "ffn_us": round(us_all, 2),
                        "ffn_tops": round((gu_ops + 2.0 * n_tok * 8960 * 1536) / us_all / 1e6, 1)}
            log(f"[bench] configs[4] prefill FFN N{n_tok} ({key}): gate/up+SwiGLU {us_gu:.1f} us, "
                f"whole FFN {us_all:.1f} us")
        dev.set_ffn_prefill_form(chart.Device.FFN_AUTO)
        # the down GEMM alone from that hidden QuantAct, and from one of biased rows' (some tokens
        # flagged: the exact path)
        down = lambda: Df.gemm_q8_dev(ptr(hcf), ptr(hsf), n_tok, ptr(yf), sh)
        ffn["down_us"] = round(event_us(down, 20), 2)
        Gb = dev.upload(synth.Q4_K, synth.payload(synth.Q4_K, rngf, 8960, 1536), 8960, 1536)
        Ub = dev.upload(synth.Q4_K, synth.payload(synth.Q4_K, rngf, 8960, 1536), 8960, 1536)
        chart.ffn_gate_up_prefill_dev(dev, Gb, Ub, ptr(xf), n_tok, ptr(hcf), ptr(hsf), None, None, sh)
        assert dev.sync_status(sh) == 0
        ffn["down_exact_path_us"] = round(event_us(down, 3), 1)
        # tokens the operand pass flags: a nonzero block more than 24 binades below the largest
        hs_np = hsf.cpu().numpy()
        e = np.log2(np.maximum(hs_np, 1).astype(np.float64))
        span = np.where(hs_np > 0, e, -np.inf).max(axis=1) - np.where(hs_np > 0, e, np.inf).min(axis=1)
        ffn["down_flagged_tokens"] = int(np.sum(span > 24))
        log(f"[bench] configs[4] prefill FFN down alone {ffn['down_us']} us; with flagged hidden tokens "
            f"{ffn['down_exact_path_us']} us ({ffn['down_flagged_tokens']} of {n_tok} tokens flagged)")
        result["ffn_prefill"] = ffn
        for w_ in (Gf, Uf, Df, Gb, Ub):
            w_.free()

    # ---- the 168 projections of a Qwen2.5-0.5B token batched in one launch ------------
    if args.only in (None, "config1") and not args.no_extras:
        t = synth.Q4_K
        layer_stored = sum(n * synth.row_bytes(t, k) for _, n, k in CFG1_SHAPES)
        n_sets = max(CFG1_LAYERS + 8, int(1.1 * (1 << 30) // layer_stored) + 1)
        host1 = [{nm: synth.payload(t, synth.rng_for(1, 100 + u), n, k) for nm, n, k in CFG1_SHAPES}
                 for u in range(4)]
        rng1 = synth.rng_for(1, 1)
        xin = {nm: torch.from_numpy(synth.activations(rng1, k)).cuda() for nm, _, k in CFG1_SHAPES}
        outs = {nm: torch.zeros(n, dtype=torch.float32, device="cuda") for nm, n, _ in CFG1_SHAPES}
        L1 = [{nm: dev.upload(t, host1[i % 4][nm], n, k) for nm, n, k in CFG1_SHAPES} for i in range(n_sets)]
        step1_bytes = CFG1_LAYERS * sum(proj_bytes(synth, t, n, k) for _, n, k in CFG1_SHAPES)
        windows = []
        for wdx in range(-(-n_sets // CFG1_LAYERS)):
            ws, xs1, ys1 = [], [], []
            for l in range(CFG1_LAYERS):
                L = L1[(wdx * CFG1_LAYERS + l) % n_sets]
                for nm, _, _ in CFG1_SHAPES:
                    ws.append(L[nm]), xs1.append(ptr(xin[nm])), ys1.append(ptr(outs[nm]))
            windows.append(chart.GemvPlan(dev, ws, xs1, ys1))
        ctr = [0]

        def step1():
            windows[ctr[0] % len(windows)].run(sh)
            ctr[0] += 1
        clock_up(step1)
        us1 = event_us(step1, 200)
        assert dev.sync_status(sh) == 0
        result["config1"] = {"us_per_token": round(us1, 2), "bytes_per_token": step1_bytes,
                             "gbs": round(step1_bytes / us1 / 1e3, 1),
                             "frac_hbm": round(step1_bytes / us1 / 1e3 / HBM_PEAK_GBS, 4),
                             "launches_per_token": 1, "pool_gib": round(n_sets * layer_stored / 2 ** 30, 2),
                             "note": "168 projections batched as independent parts in one launch"}
        log(f"[bench] configs[1] batched token: {us1:.1f} us, {step1_bytes / us1 / 1e3:.0f} GB/s")
        for p in windows:
            p.free()
        for L in L1:
            for w in L.values():
                w.free()
        del L1

    # ---- single GEMV launches over rotating copies --------------------
    if args.only in (None, "heads") and not args.no_heads and not args.no_extras:
        singles = []
        for cfg, gt, n_out, n_in in ((0, synth.Q8_0, 4864, 896), (2, synth.Q6_K, 151936, 896),
                                     (2, synth.Q8_0, 151936, 896)):
            raw = synth.payload(gt, synth.rng_for(cfg, gt), n_out, n_in)
            copies = max(2, -(-int(1.1 * 2 ** 30) // raw.nbytes))
            wc = [dev.upload(gt, raw, n_out, n_in) for _ in range(copies)]
            del raw
            x = torch.from_numpy(synth.activations(synth.rng_for(cfg, 99), n_in)).cuda()
            y = torch.empty(n_out, dtype=torch.float32, device="cuda")
            ctr = [0]

            def one():
                wc[ctr[0] % copies].gemv_f32_dev(ptr(x), ptr(y), sh)
                ctr[0] += 1
            clock_up(one, 0.05)
            assert dev.sync_status(sh) == 0
            us = event_us(one, 400 if n_out < 100000 else 60)
            nbytes = proj_bytes(synth, gt, n_out, n_in)
            gbs = nbytes / us / 1e3
            singles.append({"config": cfg, "type": synth.NAMES[gt], "shape": [n_out, n_in], "copies": copies,
                            "us": round(us, 2), "bytes": nbytes, "gbs": round(gbs, 1),
                            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)})
            log(f"[bench] configs[{cfg}] {synth.NAMES[gt]} {n_out}x{n_in}: {us:.2f} us/launch, {gbs:.0f} GB/s")
            for w in wc:
                w.free()
            del wc
        result["heads"] = singles

    # ---- the other weight families (Q5_0, Q2_K, Q3_K): a vocab-head-shaped launch (bandwidth) and a
    # configs[0]-shaped one (latency) over rotating copies, and the N = 512 GEMM at 4864x896 (Q5_0 on
    # its f16-MFMA form; Q2_K / Q3_K one GEMV launch per token, as the reference serves them)
    if args.only in (None, "families") and not args.no_heads and not args.no_extras:
        fam = []
        for gt in (synth.Q5_0, synth.Q2_K, synth.Q3_K):
            row = {"type": synth.NAMES[gt]}
            for key, n_out, n_in in (("head", 151936, 896), ("single", 4864, 896)):
                raw = synth.payload(gt, synth.rng_for(6, gt + n_out), n_out, n_in)
                copies = max(2, -(-int(1.1 * 2 ** 30) // raw.nbytes))
                wc = [dev.upload(gt, raw, n_out, n_in) for _ in range(copies)]
                del raw
                x = torch.from_numpy(synth.activations(synth.rng_for(6, 99), n_in)).cuda()
                y = torch.empty(n_out, dtype=torch.float32, device="cuda")
                ctr = [0]

                def one():
                    wc[ctr[0] % copies].gemv_f32_dev(ptr(x), ptr(y), sh)
                    ctr[0] += 1
                clock_up(one, 0.05)
                assert dev.sync_status(sh) == 0
                us = event_us(one, 400 if n_out < 100000 else 60)
                nbytes = proj_bytes(synth, gt, n_out, n_in)
                row[key] = {"shape": [n_out, n_in], "us": round(us, 2), "bytes": nbytes,
                            "gbs": round(nbytes / us / 1e3, 1), "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}
                log(f"[bench] {synth.NAMES[gt]} {n_out}x{n_in}: {us:.2f} us/launch, {nbytes / us / 1e3:.0f} GB/s")
                for w in wc:
                    w.free()
                del wc
            n_tok, n_out, n_in = 512, 4864, 896
            raw = synth.payload(gt, synth.rng_for(6, gt), n_out, n_in)
            w = dev.upload(gt, raw, n_out, n_in)
            x = torch.from_numpy(synth.activations(synth.rng_for(6, 5), n_in, n_tok).reshape(n_tok, n_in)).cuda()
            y = torch.empty((n_tok, n_out), dtype=torch.float32, device="cuda")
            run = lambda: w.gemm_f32_dev(ptr(x), n_tok, ptr(y), sh)
            clock_up(run, 0.03)
            assert dev.sync_status(sh) == 0
            us = event_us(run, 20)
            tops = 2.0 * n_tok * n_out * n_in / us / 1e6
            row["gemm"] = {"shape": [n_out, n_in], "n_tok": n_tok, "us": round(us, 2), "tops": round(tops, 1),
                           "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                           "form": "f16 MFMA" if gt == synth.Q5_0 else "f16 MFMA, dequantize-once tiles"}
            log(f"[bench] gemm {synth.NAMES[gt]} {n_out}x{n_in} N{n_tok}: {us:.1f} us {tops:.0f} TOPS")
            if gt != synth.Q5_0:
                # the per-token GEMV route (AH_GEMM_DESIGN_F16 for these families): one streaming GEMV
                # per few tokens, as the reference serves them column by column
                dev.set_gemm_design(gt, chart.Device.GEMM_F16)
                run(); torch.cuda.synchronize()
                us_g = event_us(run, 3)
                assert dev.sync_status(sh) == 0
                dev.set_gemm_design(gt, chart.Device.GEMM_AUTO)
                row["gemm"]["gemv_route_us"] = round(us_g, 1)
                log(f"[bench] gemm {synth.NAMES[gt]} per-token GEMV route: {us_g:.1f} us")
            w.free()
            fam.append(row)
        result["families"] = fam

    # ---- CPU baselines: the same token (and N = 512 sample) on the host ---------------------------
    if run_decode and not args.no_cpu:
        import oracle

        # distinct host copies of the layer payloads past the host LLC, rotated, plus the head
        n_copies = 8  # one host copy per projection of layers 0..7, rotated (~230 MB)
        copies = [{nm: host[(gt, n_out, n_in)].copy() for nm, gt, n_out, n_in in spec[i]} for i in range(n_copies)]
        xa = synth.activations(synth.rng_for(4, 2), 1536)
        xd = synth.activations(synth.rng_for(4, 3), 8960)
        st, ca, sa = oracle.quant_act_f32(xa)
        st, cd, sd = oracle.quant_act_f32(xd)

        def cpu_layer(li, threads):
            P = copies[li % n_copies]
            nbytes = 0
            for nm, gt, n_out, n_in in spec[li % n_copies]:
                c, s = (cd, sd) if n_in == 8960 else (ca, sa)
                oracle.matvec_q8act_fast(gt, P[nm], n_out, n_in, c, s, threads)
                nbytes += proj_bytes(synth, gt, n_out, n_in)
            return nbytes

        def cpu_head(threads):
            oracle.matvec_q8act_fast(synth.Q6_K, host[head_key], 151936, 1536, ca, sa, threads)
            return proj_bytes(synth, *head_key)

        runs = []
        for threads in sorted({max(1, min(args.cpu_threads, os.cpu_count() or 1)), os.cpu_count() or 1}):
            cpu_layer(0, threads)
            t0, nbytes, nl = time.perf_counter(), 0, 0
            while time.perf_counter() - t0 < args.cpu_seconds:
                nbytes += cpu_layer(nl, threads)
                nl += 1
                if nl % CFG4_LAYERS == 0:
                    nbytes += cpu_head(threads)
            el = time.perf_counter() - t0
            runs.append({"threads": threads, "gbs": round(nbytes / el / 1e9, 2), "layers": nl, "seconds": round(el, 1)})
            log(f"[bench] cpu baseline: {nbytes / el / 1e9:.1f} GB/s on {threads} threads ({nl} layers)")
        best = max(runs, key=lambda r: r["gbs"])  # the host's best: every core when that is faster
        result["cpu_baseline"] = {
            "value": best["gbs"], "unit": "GB/s", "cores": best["threads"], "kind": "port",
            "sample": f"{best['layers']} configs[4] layers ({best['layers'] / CFG4_LAYERS:.1f} tokens, the head "
                      f"once per 28 layers), f32 input quantized once per input width, {best['seconds']} s, "
                      f"{n_copies} rotating host copies of the layer payloads",
            "cpu": _cpu_name(), "host_cpus": os.cpu_count(), "cpu_flags": cpu_flags(),
            "cores_form": ("portable", "avx2", "avx_vnni")[oracle.cpu_path()], "runs": runs}
        del copies
    if args.only in (None, "gemm") and not args.no_cpu and not args.no_gemm and not args.no_extras:
        import oracle

        cg = []
        k = 512  # every token column of the configs[3] GEMMs
        thread_set = sorted({max(1, min(args.cpu_threads, os.cpu_count() or 1)), os.cpu_count() or 1})
        for gt in (synth.Q8_0, synth.Q4_K):
            for n_out, n_in in GEMM_SHAPES:
                raw = synth.payload(gt, synth.rng_for(3, gt * 10 + n_in), n_out, n_in)
                x = synth.activations(synth.rng_for(3, 5), n_in, k).reshape(k, n_in)
                st, codes, scales = oracle.quant_act_f32_batch(x)
                for threads in thread_set:
                    oracle.matmat_q8act_fast(gt, raw, n_out, n_in, codes[:2], scales[:2], threads)  # warm-up
                    reps = []
                    for _ in range(3):  # median of 3 timed calls
                        t0 = time.perf_counter()
                        oracle.matmat_q8act_fast(gt, raw, n_out, n_in, codes, scales, threads)
                        reps.append(time.perf_counter() - t0)
                    el = sorted(reps)[1]
                    gops = 2.0 * k * n_out * n_in / el / 1e9
                    cg.append({"type": synth.NAMES[gt], "shape": [n_out, n_in], "columns": k, "threads": threads,
                               "seconds": round(el, 4), "gops": round(gops, 1),
                               "route": "per-column matvec (K % 256 != 0)" if gt == synth.Q4_K and n_in % 256
                                        else "k-column",
                               "cores_form": ("portable", "avx2", "avx_vnni")[oracle.cpu_path()]})
        result["cpu_baseline_gemm"] = cg
        log(f"[bench] cpu gemm baseline: {[c['gops'] for c in cg]} GOPS")

    if not run_decode:
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
        "dtype": "int8 x Q4_K/Q6_K (exact int32 group dots, f32 fold)",
        "data": "synthetic (BASELINE.json configs[4] distributions, random-init weights, seeded)",
        "config": {"workload": "configs[4]: one decode token (N=1) of a Qwen2.5-1.5B-architecture Q4_K_M-style "
                               "model, 197 projections as 113 dependent stages (q/k/v -> o -> gate/up -> down "
                               "per layer, then the Q6_K vocab head), one HIP graph per token",
                   "parallelism": "single GPU"},
        "roofline": result["roofline"],
        "cpu_baseline": result.get("cpu_baseline"),
        "decode": result.get("decode"),
        "config4_prefill": result.get("config4_prefill"),
        "gemm": result.get("gemm"),
        "mfma_probe": result.get("mfma_probe"),
        "config1": result.get("config1"),
        "config0_config2": result.get("heads"),
        "families": result.get("families"),
        "ffn_prefill": result.get("ffn_prefill"),
        "cpu_baseline_gemm": result.get("cpu_baseline_gemm"),
    }
    print(json.dumps(line))
    dev.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
