"""Writes tests/golden/golden.npz: small fixtures computed by the big-integer brute force.

Run ``python tests/golden/make_golden.py`` from the repository root.  Each case stores the raw
GGUF payload, the Q32.32 activation (and, for f32 cases, the f32 input), the expected codes and
scales, the expected Q32.32 outputs and the exact group dots of every row -- all from
bruteforce.py, never from the oracle or the reference.  The shapes and scale words follow the
reference's own equality tests (chart/tests.rs:222-371, kern/gemm.rs:2613-2617).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import bruteforce as bf  # noqa: E402
from apeiron_amd import synth  # noqa: E402


def case_from_q32(t, raw, rows, n_in, x):
    q = bf.quant_act([int(v) for v in x])
    assert q is not None
    codes, scales = q
    xhat = [scales[i // 32] * c for i, c in enumerate(codes)]
    y = bf.matvec(t, raw.tobytes(), rows, n_in, xhat)
    rb = synth.row_bytes(t, n_in)
    dots = [bf.block_dots(t, raw[r * rb:(r + 1) * rb].tobytes(), n_in, codes) for r in range(rows)]
    return dict(t=t, rows=rows, n_in=n_in, raw=raw, x=np.asarray(x, np.int64),
                codes=np.asarray(codes, np.int8), scales=np.asarray(scales, np.int64),
                y=np.asarray(y, dtype=object), dots=np.asarray(dots, np.int64).reshape(rows, -1))


def main() -> None:
    cases = []
    rng = np.random.default_rng(0x60DE17)
    shapes = [(4, 32), (3, 48), (2, 33), (2, 300), (1, 64), (1, 256), (2, 512), (3, 896)]
    for t in (8, 12, 14):
        for rows, n_in in shapes + [(2, w) for w in (47, 65, 257, 271)]:
            raw = synth.random_bytes_payload(rng, t, rows, n_in, 0x3800, 0x3800)
            x = rng.integers(-2048, 2048, size=n_in)
            cases.append(("random", case_from_q32(t, raw, rows, n_in, x)))
        # BASELINE-style payload with f32 N(0,1) activations
        raw = synth.payload(t, rng, 3, 896)
        xf = rng.standard_normal(896).astype(np.float32)
        xq = [bf.f32_q32(int(w)) for w in xf.view(np.uint32)]
        c = case_from_q32(t, raw, 3, 896, xq)
        c["xf"] = xf
        cases.append(("f32", c))
        # extremes: largest finite scale, +-127 codes at unit scale
        raw = synth.random_bytes_payload(rng, t, 2, 256, 0x7BFF, 0x7BFF)
        x = [127 if j % 2 == 0 else -127 for j in range(256)]
        cases.append(("extreme", case_from_q32(t, raw, 2, 256, x)))
        # zero activation blocks
        x = [0] * 64 + [1000 - 100 * j for j in range(64, 96)]
        raw = synth.random_bytes_payload(rng, t, 1, 96, 0x3800, 0x3800)
        cases.append(("zeroblk", case_from_q32(t, raw, 1, 96, x)))
    # Q8_0 scale-word sets and wide activation spreads (kern/gemm.rs:2613-2617, :2490-2506)
    for words in ([0x2000, 0x2400, 0x1C00, 0xA000], [0x0001, 0x03FF, 0x0400, 0x8200],
                  [0x0000, 0x3C00, 0x0010, 0x7BFF]):
        for bits in (1, 8, 30):
            raw = rng.integers(0, 256, size=(4 * 3, 34), dtype=np.uint8)
            w = rng.choice(words, size=4 * 3)
            raw[:, 0], raw[:, 1] = w & 0xFF, w >> 8
            raw = raw.reshape(-1)
            mags = 1 << (20 + rng.integers(0, bits, size=96))
            x = [int(rng.integers(-m, m + 1)) if (j // 32) % 7 != 3 else 0 for j, m in enumerate(mags.tolist())]
            c = case_from_q32(8, raw, 4, 96, x)
            if all(-(1 << 63) <= v < (1 << 63) for v in c["y"]):
                cases.append(("scaleset", c))
    # Q5_0 (format/quant.rs:261-297), appended with a stream of its own so the cases above keep
    # their bytes: the same shape families, random qh/qs bytes, BASELINE-style payloads with f32
    # N(0,1) input, the largest finite scale against +-127 codes, zero activation blocks
    rng5 = np.random.default_rng(0x60DE50)
    for rows, n_in in shapes + [(2, w) for w in (47, 65, 257, 271)]:
        raw = synth.random_bytes_payload(rng5, 6, rows, n_in, 0x3800, 0x3800)
        x = rng5.integers(-2048, 2048, size=n_in)
        cases.append(("random", case_from_q32(6, raw, rows, n_in, x)))
    raw = synth.payload(6, rng5, 3, 896)
    xf = rng5.standard_normal(896).astype(np.float32)
    c = case_from_q32(6, raw, 3, 896, [bf.f32_q32(int(w)) for w in xf.view(np.uint32)])
    c["xf"] = xf
    cases.append(("f32", c))
    raw = synth.random_bytes_payload(rng5, 6, 2, 256, 0x7BFF, 0x7BFF)
    cases.append(("extreme", case_from_q32(6, raw, 2, 256, [127 if j % 2 == 0 else -127 for j in range(256)])))
    raw = synth.random_bytes_payload(rng5, 6, 1, 96, 0x3800, 0x3800)
    cases.append(("zeroblk", case_from_q32(6, raw, 1, 96, [0] * 64 + [1000 - 100 * j for j in range(64, 96)])))
    # Q2_K and Q3_K (format/quant.rs:308-476), each with a stream of its own: the same families
    for t, seed in ((10, 0x60DE10), (11, 0x60DE11)):
        rk = np.random.default_rng(seed)
        for rows, n_in in shapes + [(2, w) for w in (47, 65, 257, 271)]:
            raw = synth.random_bytes_payload(rk, t, rows, n_in, 0x3800, 0x3400)
            x = rk.integers(-2048, 2048, size=n_in)
            cases.append(("random", case_from_q32(t, raw, rows, n_in, x)))
        raw = synth.payload(t, rk, 3, 896)
        xf = rk.standard_normal(896).astype(np.float32)
        c = case_from_q32(t, raw, 3, 896, [bf.f32_q32(int(w)) for w in xf.view(np.uint32)])
        c["xf"] = xf
        cases.append(("f32", c))
        raw = synth.random_bytes_payload(rk, t, 2, 256, 0x7BFF, 0x7BFF)
        cases.append(("extreme", case_from_q32(t, raw, 2, 256, [127 if j % 2 == 0 else -127 for j in range(256)])))
        raw = synth.random_bytes_payload(rk, t, 1, 96, 0x3800, 0x3800)
        cases.append(("zeroblk", case_from_q32(t, raw, 1, 96, [0] * 64 + [1000 - 100 * j for j in range(64, 96)])))
    out = {}
    for i, (kind, c) in enumerate(cases):
        p = f"c{i:03d}_"
        out[p + "meta"] = np.array([c["t"], c["rows"], c["n_in"]], np.int64)
        out[p + "kind"] = np.array(kind)
        out[p + "raw"] = c["raw"]
        out[p + "x"] = c["x"]
        out[p + "codes"] = c["codes"]
        out[p + "scales"] = c["scales"]
        out[p + "y"] = np.array([int(v) for v in c["y"]], np.int64)
        out[p + "dots"] = c["dots"].astype(np.int32)
        if "xf" in c:
            out[p + "xf"] = c["xf"]
    out["count"] = np.array(len(cases), np.int64)
    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {len(cases)} cases to {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
