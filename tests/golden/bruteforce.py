"""Independent big-integer brute force of the projection contract (this project's own code).

Used to pin the C oracle: every quantity is derived from first principles with Python's
unbounded integers and ``fractions.Fraction`` -- the f16 and f32 values come from numpy's
IEEE conversions (exact in float64), not from any bit-level decode shared with the oracle.

* f16 scale      -> exact real value * 2^32 (an integer for every finite f16)
* f32 activation -> round-half-away(v * 2^32)
* act scale      -> the least power of two S with 127*S >= absmax (searched, not computed)
* codes          -> round-half-away(x / S)
* weights        -> the documented GGUF formulas on exact values
* output         -> floor((sum w*xhat + 2^31) / 2^32)
"""
from __future__ import annotations

from fractions import Fraction
import math

import numpy as np

TWO32 = 1 << 32


def f16_value(word: int) -> Fraction | None:
    v = np.array([word], dtype=np.uint16).view(np.float16)[0]
    if not np.isfinite(v):
        return None
    return Fraction(float(v))


def f16_q32(word: int) -> int | None:
    v = f16_value(word)
    if v is None:
        return None
    q = v * TWO32
    assert q.denominator == 1
    return int(q)


def round_half_away(fr: Fraction) -> int:
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    fl = math.floor(a)
    if a - fl >= Fraction(1, 2):
        fl += 1
    return sign * fl


def f32_q32(bits: int) -> int | None:
    v = np.array([bits], dtype=np.uint32).view(np.float32)[0]
    if not np.isfinite(v):
        return None
    q = round_half_away(Fraction(float(v)) * TWO32)
    if q < -(1 << 63) or q >= (1 << 63):
        return None
    return q


def least_pow2_scale(absmax: int) -> int | None:
    if absmax == 0:
        return 0
    s = 1
    while 127 * s < absmax:
        s *= 2
        if s > (1 << 62):
            return None
    return s


def quant_act(x: list[int]):
    codes, scales = [], []
    for b in range(0, len(x), 32):
        blk = x[b:b + 32]
        s = least_pow2_scale(max(abs(v) for v in blk))
        if s is None:
            return None
        scales.append(s)
        for v in blk:
            c = 0 if s == 0 else round_half_away(Fraction(v, s))
            if abs(c) > 127:
                return None
            codes.append(c)
    for i, c in enumerate(codes):
        if not -(1 << 63) <= scales[i // 32] * c < (1 << 63):
            return None
    return codes, scales


def q4k_pairs(sc12: bytes) -> list[tuple[int, int]]:
    """Sub-block (scale, min) pairs by the ggml packing rule, written from the format notes."""
    out = []
    for j in range(8):
        if j < 4:
            out.append((sc12[j] & 63, sc12[j + 4] & 63))
        else:
            lo = sc12[j + 4]
            out.append(((lo & 0xF) | ((sc12[j - 4] >> 6) << 4), (lo >> 4) | ((sc12[j] >> 6) << 4)))
    return out


def q5_0_codes(blk: bytes) -> list[int]:
    """A Q5_0 block's 32 codes minus 16: element e < 16 is qs[e] & 15 with the fifth bit from bit e of
    the little-endian word qh = blk[2:6]; element 16 + e is qs[e] >> 4 with bit 16 + e."""
    qh = int.from_bytes(blk[2:6], "little")
    qs = blk[6:22]
    lo = [(qs[e] & 15) + 16 * ((qh >> e) & 1) - 16 for e in range(16)]
    hi = [(qs[e] >> 4) + 16 * ((qh >> (16 + e)) & 1) - 16 for e in range(16)]
    return lo + hi


def k23_position(e: int) -> tuple[int, int, int]:
    """Where Q2_K / Q3_K element e (0..255) sits: the qs byte index, the bit shift of its two bits,
    and the bit of the hmask byte (16 * plane + l) that carries Q3_K's third bit.  Elements run in
    two halves of 128; a half is four rounds of 32 (each round one bit pair of every qs byte of the
    half), a round two planes of 16 consecutive qs bytes."""
    half, r = divmod(e, 128)
    rnd, r = divmod(r, 32)
    plane, l = divmod(r, 16)
    return 32 * half + 16 * plane + l, 2 * rnd, 4 * half + rnd


def q2k_codes(blk: bytes) -> list[int]:
    """The 256 two-bit Q2_K values 0..3 (qs at byte 16)."""
    out = []
    for e in range(256):
        i, sh, _ = k23_position(e)
        out.append((blk[16 + i] >> sh) & 3)
    return out


def q3k_codes(blk: bytes) -> list[int]:
    """The 256 signed Q3_K codes: the two qs bits (qs at byte 32) minus 4 unless the hmask bit is set."""
    out = []
    for e in range(256):
        i, sh, hb = k23_position(e)
        q = (blk[32 + i] >> sh) & 3
        h = (blk[e % 32] >> hb) & 1
        out.append(q - (0 if h else 4))
    return out


def q3k_scales(sc12: bytes) -> list[int]:
    """The sixteen 6-bit Q3_K group scales: low four bits from the nibbles of bytes 0..7 (group j < 8
    the low nibble of byte j, group j >= 8 the high nibble of byte j - 8), high two bits from bit pair
    j // 4 of byte 8 + j % 4."""
    out = []
    for j in range(16):
        lo = (sc12[j] & 0xF) if j < 8 else (sc12[j - 8] >> 4)
        hi = (sc12[8 + j % 4] >> (2 * (j // 4))) & 3
        out.append(lo | (hi << 4))
    return out


def weights_row(ggml_type: int, row: bytes, n: int) -> list[int] | None:
    """Exact Q32.32 weights of one row, or None for a non-finite scale."""
    w: list[int] = []
    if ggml_type == 8:
        for b in range(-(-n // 32)):
            blk = row[34 * b:34 * b + 34]
            d = f16_q32(blk[0] | (blk[1] << 8))
            if d is None:
                return None
            w += [d * (c - 256 if c > 127 else c) for c in blk[2:34]]
    elif ggml_type == 6:
        for b in range(-(-n // 32)):
            blk = row[22 * b:22 * b + 22]
            d = f16_q32(blk[0] | (blk[1] << 8))
            if d is None:
                return None
            w += [d * c for c in q5_0_codes(blk)]
    elif ggml_type == 12:
        for s in range(-(-n // 256)):
            blk = row[144 * s:144 * s + 144]
            d, dm = f16_q32(blk[0] | (blk[1] << 8)), f16_q32(blk[2] | (blk[3] << 8))
            if d is None or dm is None:
                return None
            pairs = q4k_pairs(blk[4:16])
            vals = [0] * 256
            for j in range(8):
                sc, m = pairs[j]
                for l in range(32):
                    byte = blk[16 + 32 * (j // 2) + l]
                    q = (byte >> 4) if j % 2 else (byte & 0xF)
                    vals[32 * j + l] = d * sc * q - dm * m
            w += vals
    elif ggml_type == 10:
        for s in range(-(-n // 256)):
            blk = row[84 * s:84 * s + 84]
            d, dm = f16_q32(blk[80] | (blk[81] << 8)), f16_q32(blk[82] | (blk[83] << 8))
            if d is None or dm is None:
                return None
            q = q2k_codes(blk)
            w += [d * (blk[e // 16] & 0xF) * q[e] - dm * (blk[e // 16] >> 4) for e in range(256)]
    elif ggml_type == 11:
        for s in range(-(-n // 256)):
            blk = row[110 * s:110 * s + 110]
            d = f16_q32(blk[108] | (blk[109] << 8))
            if d is None:
                return None
            c, sc = q3k_codes(blk), q3k_scales(blk[96:108])
            w += [d * (sc[e // 16] - 32) * c[e] for e in range(256)]
    elif ggml_type == 14:
        for s in range(-(-n // 256)):
            blk = row[210 * s:210 * s + 210]
            d = f16_q32(blk[208] | (blk[209] << 8))
            if d is None:
                return None
            vals = [0] * 256
            for e in range(256):
                half, r = divmod(e, 128)
                t, l = divmod(r, 32)
                qlb = blk[64 * half + l + 32 * (t & 1)]
                lo = (qlb & 0xF) if t < 2 else (qlb >> 4)
                hi = (blk[128 + 32 * half + l] >> (2 * t)) & 3
                sc = blk[192 + e // 16]
                sc = sc - 256 if sc > 127 else sc
                vals[e] = d * sc * ((lo | (hi << 4)) - 32)
            w += vals
    else:
        raise ValueError(ggml_type)
    return w[:n]


def matvec(ggml_type: int, raw: bytes, n_out: int, n_in: int, xhat: list[int]):
    """floor((sum w*xhat + 2^31) / 2^32) per row, or None on a refusal."""
    rb = {6: 22 * -(-n_in // 32), 8: 34 * -(-n_in // 32), 10: 84 * -(-n_in // 256), 11: 110 * -(-n_in // 256),
          12: 144 * -(-n_in // 256), 14: 210 * -(-n_in // 256)}[ggml_type]
    ys = []
    for o in range(n_out):
        w = weights_row(ggml_type, raw[o * rb:(o + 1) * rb], n_in)
        if w is None:
            return None
        acc = sum(a * b for a, b in zip(w, xhat))
        ys.append((acc + (1 << 31)) >> 32)
    return ys


def block_dots(ggml_type: int, row: bytes, n_in: int, codes: list[int]):
    """Exact integer group dots: per-32 (Q8_0 codes, Q5_0 q-16, Q4_K nibbles), per-16 (Q6_K u-32,
    Q2_K's two-bit values, Q3_K's signed codes)."""
    w_codes: list[int] = []
    if ggml_type == 8:
        for b in range(-(-n_in // 32)):
            w_codes += [c - 256 if c > 127 else c for c in row[34 * b + 2:34 * b + 34]]
        g = 32
    elif ggml_type == 6:
        for b in range(-(-n_in // 32)):
            w_codes += q5_0_codes(row[22 * b:22 * b + 22])
        g = 32
    elif ggml_type == 12:
        for s in range(-(-n_in // 256)):
            blk = row[144 * s:144 * s + 144]
            for j in range(8):
                for l in range(32):
                    byte = blk[16 + 32 * (j // 2) + l]
                    w_codes.append((byte >> 4) if j % 2 else (byte & 0xF))
        g = 32
    elif ggml_type in (10, 11):
        bb = 84 if ggml_type == 10 else 110
        for s in range(-(-n_in // 256)):
            blk = row[bb * s:bb * s + bb]
            w_codes += q2k_codes(blk) if ggml_type == 10 else q3k_codes(blk)
        g = 16
    else:
        for s in range(-(-n_in // 256)):
            blk = row[210 * s:210 * s + 210]
            for e in range(256):
                half, r = divmod(e, 128)
                t, l = divmod(r, 32)
                qlb = blk[64 * half + l + 32 * (t & 1)]
                lo = (qlb & 0xF) if t < 2 else (qlb >> 4)
                hi = (blk[128 + 32 * half + l] >> (2 * t)) & 3
                w_codes.append((lo | (hi << 4)) - 32)
        g = 16
    dots = []
    for b in range(-(-n_in // g)):
        dots.append(sum(w_codes[i] * codes[i] for i in range(b * g, min(n_in, b * g + g))))
    return dots
