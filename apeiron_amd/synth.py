"""Seeded synthetic GGUF payloads and activations for the quantized-projection path.

The generators build raw GGUF block bytes exactly as the reference reads them
(format/quant.rs:238-250 Q8_0, :481-510 Q4_K, :556-599 Q6_K) from the distributions of the
benchmark configurations:

* Q8_0: codes uniform in [-127, 127]; block scale d = f16(|N(0, sigma)| / 127).
* Q4_K: nibbles uniform 0..15; 6-bit sub-block scales and mins uniform 0..63;
  d and dmin = f16(|N(0, 0.01)|).  A ragged row (K % 256 != 0) still stores whole
  super-blocks; their unused tail is random and must be ignored by every kernel.
* Q6_K: 6-bit quants uniform 0..63; int8 16-group scales uniform in [-128, 127];
  d = f16(|N(0, 0.01)|).
* Q2_K / Q3_K (format/quant.rs:308-476): every code, scale and mask byte uniform 0..255;
  d (and Q2_K's dmin) = f16(|N(0, 0.01)|).
* Activations: f32 N(0, 1).

f16 rounding is numpy's float16 conversion (round to nearest even).  The RNG is numpy's
PCG64 seeded with ``0x5EED0000 + config_index`` plus a per-tensor stream index.
"""
from __future__ import annotations

import numpy as np

Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q6_K = 6, 8, 10, 11, 12, 14
GEOM = {Q5_0: (32, 22), Q8_0: (32, 34), Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144), Q6_K: (256, 210)}
NAMES = {Q5_0: "Q5_0", Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q6_K: "Q6_K"}
# f16 scale words of a block: (byte offset of d, byte offset of dmin or None)
SCALE_AT = {Q5_0: (0, None), Q8_0: (0, None), Q2_K: (80, 82), Q3_K: (108, None), Q4_K: (0, 2), Q6_K: (208, None)}


def row_bytes(ggml_type: int, n_in: int) -> int:
    qk, bb = GEOM[ggml_type]
    return -(-n_in // qk) * bb


def needed_row_bytes(ggml_type: int, n_in: int) -> int:
    """Bytes of one row a correct kernel must read (the algorithmic traffic per row)."""
    if ggml_type in (Q8_0, Q5_0):
        return GEOM[ggml_type][1] * (-(-n_in // 32))
    full, rem = divmod(n_in, 256)
    if ggml_type == Q4_K:
        # header 16 B + the qs bytes of the used sub-block pairs
        tail = 0 if rem == 0 else 16 + 32 * (-(-rem // 64))
        return 144 * full + tail
    if ggml_type in (Q2_K, Q3_K):
        # a used half (128 elements) reads its 32 qs bytes; the rest of the block is read whole
        # (Q2_K: scales 16 + d/dmin 4; Q3_K: hmask 32 + scales 12 + d 2)
        other = 20 if ggml_type == Q2_K else 46
        return GEOM[ggml_type][1] * full + (0 if rem == 0 else other + 32 * (-(-rem // 128)))
    # Q6_K: ql + qh + sc of the used halves + d
    if rem == 0:
        return 210 * full
    halves = -(-rem // 128)
    return 210 * full + halves * (64 + 32 + 8) + 2


def rng_for(config: int, stream: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([0x5EED0000 + config, stream]))


def _f16_abs_normal(rng: np.random.Generator, n: int, sigma: float, div: float = 1.0) -> np.ndarray:
    v = np.abs(rng.standard_normal(n)) * sigma / div
    return v.astype(np.float16).view(np.uint16)


def q8_0_payload(rng: np.random.Generator, rows: int, n_in: int, sigma: float = 0.02) -> np.ndarray:
    nb = -(-n_in // 32)
    blk = np.empty((rows * nb, 34), dtype=np.uint8)
    d = _f16_abs_normal(rng, rows * nb, sigma, 127.0)
    blk[:, 0] = d & 0xFF
    blk[:, 1] = d >> 8
    blk[:, 2:] = rng.integers(-127, 128, size=(rows * nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
    return blk.reshape(-1)


def q5_0_payload(rng: np.random.Generator, rows: int, n_in: int, sigma: float = 0.02) -> np.ndarray:
    """Q5_0 blocks (format/quant.rs:261-297): f16 d = |N(0, sigma)| / 16, random qh and qs bytes
    (every five-bit code 0..31 equally likely)."""
    nb = -(-n_in // 32)
    blk = np.empty((rows * nb, 22), dtype=np.uint8)
    d = _f16_abs_normal(rng, rows * nb, sigma, 16.0)
    blk[:, 0] = d & 0xFF
    blk[:, 1] = d >> 8
    blk[:, 2:] = rng.integers(0, 256, size=(rows * nb, 20), dtype=np.uint8)
    return blk.reshape(-1)


def pack_q4_k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Inverse of ggml get_scale_min_k4 (format/quant.rs:482-491): (n, 8) 6-bit pairs -> (n, 12)."""
    sc = sc.astype(np.uint8)
    m = m.astype(np.uint8)
    out = np.empty((sc.shape[0], 12), dtype=np.uint8)
    out[:, 0:4] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = (m[:, 0:4] & 63) | ((m[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 0xF) | ((m[:, 4:8] & 0xF) << 4)
    return out


def q4_k_payload(rng: np.random.Generator, rows: int, n_in: int, sigma: float = 0.01) -> np.ndarray:
    nsb = -(-n_in // 256)
    n = rows * nsb
    blk = np.empty((n, 144), dtype=np.uint8)
    d = _f16_abs_normal(rng, n, sigma)
    dm = _f16_abs_normal(rng, n, sigma)
    blk[:, 0] = d & 0xFF
    blk[:, 1] = d >> 8
    blk[:, 2] = dm & 0xFF
    blk[:, 3] = dm >> 8
    sc = rng.integers(0, 64, size=(n, 8))
    m = rng.integers(0, 64, size=(n, 8))
    blk[:, 4:16] = pack_q4_k_scales(sc, m)
    nib = rng.integers(0, 16, size=(n, 256), dtype=np.uint8)
    # output order: 4 windows of (32 low nibbles, 32 high nibbles) over qs[32*w + l]
    nib = nib.reshape(n, 4, 2, 32)
    blk[:, 16:] = (nib[:, :, 0, :] | (nib[:, :, 1, :] << 4)).reshape(n, 128)
    return blk.reshape(-1)


def q4_k_centered_payload(rng: np.random.Generator, rows: int, n_in: int, sigma: float = 0.01) -> np.ndarray:
    """Q4_K super-blocks whose weights average about zero (dmin = d, m = round(7.5 sc), sc in
    1..8): rows without the common positive bias of q4_k_payload, whose projections of a token
    then share its sign and make SwiGLU hidden vectors with far smaller blocks than their
    largest (tokens the GEMM's f16 band cannot carry)."""
    raw = q4_k_payload(rng, rows, n_in, sigma)
    blk = raw.reshape(-1, 144)
    n = blk.shape[0]
    sc = rng.integers(1, 9, size=(n, 8))
    blk[:, 2:4] = blk[:, 0:2]
    blk[:, 4:16] = pack_q4_k_scales(sc, np.minimum(63, np.round(sc * 7.5)).astype(np.int64))
    return raw


def pack_q6_k_codes(u: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Inverse of q6_k_codes (format/quant.rs:574-599): (n, 256) values 0..63 -> ql (n,128), qh (n,64)."""
    u = u.astype(np.uint8).reshape(-1, 2, 4, 32)  # [n][half][t][l]
    ql = np.empty((u.shape[0], 2, 2, 32), dtype=np.uint8)
    ql[:, :, 0, :] = (u[:, :, 0, :] & 0xF) | ((u[:, :, 2, :] & 0xF) << 4)
    ql[:, :, 1, :] = (u[:, :, 1, :] & 0xF) | ((u[:, :, 3, :] & 0xF) << 4)
    qh = ((u[:, :, 0, :] >> 4) | ((u[:, :, 1, :] >> 4) << 2) | ((u[:, :, 2, :] >> 4) << 4)
          | ((u[:, :, 3, :] >> 4) << 6)).astype(np.uint8)
    return ql.reshape(-1, 128), qh.reshape(-1, 64)


def q6_k_payload(rng: np.random.Generator, rows: int, n_in: int, sigma: float = 0.01) -> np.ndarray:
    nsb = -(-n_in // 256)
    n = rows * nsb
    blk = np.empty((n, 210), dtype=np.uint8)
    u = rng.integers(0, 64, size=(n, 256), dtype=np.uint8)
    ql, qh = pack_q6_k_codes(u)
    blk[:, 0:128] = ql
    blk[:, 128:192] = qh
    blk[:, 192:208] = rng.integers(-128, 128, size=(n, 16), dtype=np.int16).astype(np.int8).view(np.uint8)
    d = _f16_abs_normal(rng, n, sigma)
    blk[:, 208] = d & 0xFF
    blk[:, 209] = d >> 8
    return blk.reshape(-1)


def q23_k_payload(ggml_type: int, rng: np.random.Generator, rows: int, n_in: int,
                  sigma: float = 0.01) -> np.ndarray:
    """Q2_K / Q3_K super-blocks: random code, scale and mask bytes, f16 d (and dmin) = |N(0, sigma)|."""
    bb = GEOM[ggml_type][1]
    n = rows * (-(-n_in // 256))
    blk = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
    od, om = SCALE_AT[ggml_type]
    for o in (od, om):
        if o is not None:
            w = _f16_abs_normal(rng, n, sigma)
            blk[:, o], blk[:, o + 1] = w & 0xFF, w >> 8
    return blk.reshape(-1)


def payload(ggml_type: int, rng: np.random.Generator, rows: int, n_in: int) -> np.ndarray:
    if ggml_type in (Q2_K, Q3_K):
        return q23_k_payload(ggml_type, rng, rows, n_in)
    if ggml_type == Q8_0:
        return q8_0_payload(rng, rows, n_in)
    if ggml_type == Q5_0:
        return q5_0_payload(rng, rows, n_in)
    if ggml_type == Q4_K:
        return q4_k_payload(rng, rows, n_in)
    if ggml_type == Q6_K:
        return q6_k_payload(rng, rows, n_in)
    raise ValueError(f"unsupported ggml type {ggml_type}")


def random_bytes_payload(rng: np.random.Generator, ggml_type: int, rows: int, n_in: int,
                         d: int, dmin: int) -> np.ndarray:
    """Random block bytes with every f16 scale word overwritten (chart/tests.rs:25-70 shape)."""
    qk, bb = GEOM[ggml_type]
    nblk = rows * (-(-n_in // qk))
    raw = rng.integers(0, 256, size=(nblk, bb), dtype=np.uint8)
    od, om = SCALE_AT[ggml_type]
    raw[:, od], raw[:, od + 1] = d & 0xFF, d >> 8
    if om is not None:
        raw[:, om], raw[:, om + 1] = dmin & 0xFF, dmin >> 8
    return raw.reshape(-1)


def activations(rng: np.random.Generator, n: int, n_tok: int = 1) -> np.ndarray:
    x = rng.standard_normal((n_tok, n)).astype(np.float32)
    return x[0] if n_tok == 1 else x
