"""f32 activations built around the quantizer's rounding edges, shared by the CPU identity tests
and the GPU parity tests (no oracle or device code here: inputs only).

Blocks of 32 elements:
* a sweep of block maxima from 2^-60 to 2^23, each with elements down to 40 binades below it,
  signed zeros, the smallest subnormal, and the two neighbours of 2^-9 (where to_q32 starts
  rounding);
* largest magnitudes 1/4 (exponent 24) and 0.499 (exponent 25) with 2^-9 (1 - 2^-24), whose
  Q32.32 value 2^23 - 1/2 rounds to 2^23 before the code;
* the element just below half a code unit, 2^(e-33) (1 - 2^-24), for exponents 25, 30, 43, 54
  (v = 1/2 - 2^-25, which an f32 sum v + 1/2 rounds up to 1);
* the exponent's mantissa boundary (0xFE0000 vs 0xFE0001 with the hidden bit) at every biased
  exponent 118..155;
* blocks outside the f32 fast form's range: largest magnitude below 2^-9, and in [2^29, 2^31);
* a zero block and N(0, 1) blocks.
"""
import numpy as np


def edge_blocks_f32(rng: np.random.Generator, normal_blocks: int = 400) -> np.ndarray:
    blocks = []
    for top in list(range(-60, 24)) + [-126, -149]:
        amax = np.float32(np.ldexp(1.0 + rng.random(), top)) if top > -149 else np.float32(np.ldexp(1.0, -149))
        for _ in range(6):
            rel = rng.integers(-40, 1, size=31)
            body = np.ldexp(rng.random(31) + 0.5, top + rel).astype(np.float32)
            body *= np.where(rng.random(31) < 0.5, -1, 1).astype(np.float32)
            body[0] = np.float32(np.ldexp(1.5, top - 6))
            body[1] = np.float32(np.ldexp(0.5, -32))
            body[2] = np.float32(-np.ldexp(1.5, -33))
            body[3] = np.float32(0.0)
            body[4] = np.float32(-0.0)
            body[5] = np.float32(np.ldexp(1.0, -149))
            body[6] = np.float32(np.ldexp(1.0, -9) * (1 - 2 ** -24))
            body[7] = np.float32(-np.ldexp(1.0, -9))
            blocks.append(np.concatenate([[amax], body]).astype(np.float32))
    for amax in (0.25, -0.25, 0.499, 0.4375):
        for sgn in (1, -1):
            b = np.zeros(32, np.float32)
            b[0] = amax
            b[1] = sgn * np.float32(np.ldexp(1.0, -9) * (1 - 2 ** -24))
            b[2] = sgn * np.float32(np.ldexp(1.0, -10))
            blocks.append(b)
    for amax, e in ((0.75, 25), (24.0, 30), (1.5 * 2.0 ** 17, 43), (1.9 * 2.0 ** 28, 54)):
        b = np.zeros(32, np.float32)
        b[0] = np.float32(amax)
        b[3] = np.float32(np.ldexp(1.0, e - 33) * (1 - 2 ** -24))
        b[4] = -b[3]
        b[5] = np.float32(np.ldexp(1.0, e - 33))
        b[6] = np.float32(-np.ldexp(1.0, e - 33))
        blocks.append(b)
    for ee in range(118, 156):
        for m in (0, 1, 0x7DFFFF, 0x7E0000, 0x7E0001, 0x7FFFFF):
            b = np.zeros(32, np.uint32)
            b[5] = (ee << 23) | m
            b[9] = ((ee - 3) << 23) | 0x80000000 | m
            blocks.append(b.view(np.float32))
    for amax in (np.ldexp(1.0, -10), np.ldexp(1.5, -20), 2.0 ** 29, -1.9 * 2.0 ** 30):
        b = (rng.standard_normal(32) * (abs(amax) / 8)).astype(np.float32)
        b[7] = np.float32(amax)
        blocks.append(b)
    blocks.append(np.zeros(32, np.float32))
    blocks.append(rng.standard_normal(32 * normal_blocks).astype(np.float32))
    return np.concatenate(blocks).astype(np.float32)
