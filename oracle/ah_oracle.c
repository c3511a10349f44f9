/*
 * ah_oracle.c -- exact CPU restatement of apeiron's quantized-projection contract.
 *
 * TEST INFRASTRUCTURE ONLY (see ah_oracle.h).  Every value here is exact integer
 * arithmetic in int64 / __int128, as in the reference; nothing rounds except the
 * single round_shift_32 epilogue (num/value.rs:9-12).
 */
#include "ah_oracle.h"

#include <stdlib.h>
#include <string.h>

typedef __int128 i128;
typedef unsigned __int128 u128;

#define QK_K 256
#define Q8_0_BYTES 34
#define Q5_0_BYTES 22
#define Q2_K_BYTES 84
#define Q3_K_BYTES 110
#define Q4_K_BYTES 144
#define Q6_K_BYTES 210

/* format/quant.rs:129-147 (the three path families). */
int aho_block_geom(uint32_t t, size_t *qk, size_t *bb) {
    switch (t) {
    case AHO_Q8_0: *qk = 32; *bb = Q8_0_BYTES; return 1;
    case AHO_Q5_0: *qk = 32; *bb = Q5_0_BYTES; return 1;
    case AHO_Q2_K: *qk = QK_K; *bb = Q2_K_BYTES; return 1;
    case AHO_Q3_K: *qk = QK_K; *bb = Q3_K_BYTES; return 1;
    case AHO_Q4_K: *qk = QK_K; *bb = Q4_K_BYTES; return 1;
    case AHO_Q6_K: *qk = QK_K; *bb = Q6_K_BYTES; return 1;
    default: return 0;
    }
}

int aho_row_bytes(uint32_t t, size_t n_in, size_t *row_bytes) {
    size_t qk, bb;
    if (!aho_block_geom(t, &qk, &bb)) return AHO_ERR_UNSUPPORTED_QUANT;
    size_t blocks = n_in / qk + (n_in % qk != 0);
    if (__builtin_mul_overflow(blocks, bb, row_bytes)) return AHO_ERR_LENGTH_OVERFLOW;
    return AHO_OK;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* num/dequant.rs:25-41: subnormal m<<8, normal (1024+m)<<(e+7), Inf/NaN refuse. */
int aho_f16_to_fixed(uint16_t h, int64_t *out) {
    unsigned sign = h >> 15, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    int64_t mag;
    if (e == 0) {
        mag = (int64_t)m << 8;
    } else if (e == 0x1f) {
        return AHO_ERR_NONFINITE_SCALE;
    } else {
        mag = ((int64_t)m + 1024) << (e + 7); /* < 2^11 * 2^37 = 2^48: no overflow */
    }
    *out = sign ? -mag : mag;
    return AHO_OK;
}

/* num/fp.rs:186-230: round_half_away(v * 2^32) from the f32 fields; f32_convert.rs:44-49
 * splits the refusal into NonFinite and OutOfRange. */
int aho_to_q32(uint32_t bits, int64_t *out) {
    uint32_t e = (bits >> 23) & 0xff;
    if (e == 0xff) return AHO_ERR_NONFINITE_INPUT;
    uint32_t frac = bits & 0x7fffffu;
    uint64_t m = e == 0 ? frac : (frac | 0x800000u);
    int neg = (bits >> 31) & 1;
    uint32_t ee = e == 0 ? 1 : e;
    u128 mag;
    if (ee >= 118) {
        uint32_t k = ee - 118;
        if (k > 40) return AHO_ERR_INPUT_RANGE;
        mag = (u128)m << k;
    } else {
        uint32_t sh = 118 - ee;
        mag = sh > 24 ? 0 : (u128)((m + (1ull << (sh - 1))) >> sh);
    }
    const u128 lim = (u128)1 << 63;
    if (neg) {
        if (mag > lim) return AHO_ERR_INPUT_RANGE;
        *out = mag == lim ? INT64_MIN : -(int64_t)mag;
    } else {
        if (mag >= lim) return AHO_ERR_INPUT_RANGE;
        *out = (int64_t)mag;
    }
    return AHO_OK;
}

/* kern/pow2.rs:11-39: smallest power of two S with 127*S >= absmax (0 for 0), None past 2^62. */
int aho_act_scale(uint64_t absmax, uint64_t *out) {
    if (absmax == 0) {
        *out = 0;
        return 0;
    }
    uint64_t need = absmax / 127 + (absmax % 127 != 0);
    uint64_t s = 1;
    unsigned steps = 0;
    while (s < need && steps < 62) {
        s *= 2;
        steps++;
    }
    if (s < need) return 1;
    *out = s;
    return 0;
}

static inline uint64_t uabs64(int64_t v) { return v < 0 ? (uint64_t)0 - (uint64_t)v : (uint64_t)v; }

/* QuantAct::dequantizes (chart/mod.rs:105-134). */
static int dequantizes(const int8_t *codes, const int64_t *scales, size_t n) {
    size_t nb = (n + 31) / 32;
    for (size_t b = 0; b < nb; b++) {
        int64_t s = scales[b], p;
        if (__builtin_mul_overflow(s, (int64_t)127, &p)) {
            size_t end = (b + 1) * 32 < n ? (b + 1) * 32 : n;
            for (size_t l = b * 32; l < end; l++)
                if (__builtin_mul_overflow(s, (int64_t)codes[l], &p)) return 0;
        }
    }
    return 1;
}

/* chart/mod.rs:258-334. */
int aho_quant_act(const int64_t *x, size_t n, int8_t *codes, int64_t *scales) {
    size_t nb = (n + 31) / 32;
    for (size_t b = 0; b < nb; b++) {
        size_t base = b * 32, take = n - base < 32 ? n - base : 32;
        uint64_t absmax = 0;
        for (size_t l = 0; l < take; l++) {
            uint64_t m = uabs64(x[base + l]);
            if (m > absmax) absmax = m;
        }
        uint64_t s;
        if (aho_act_scale(absmax, &s)) s = UINT64_MAX;
        if (s > (uint64_t)INT64_MAX) return AHO_ERR_FIXED_OVERFLOW;
        scales[b] = (int64_t)s;
        for (size_t l = 0; l < take; l++) {
            int64_t v = x[base + l];
            int code = 0;
            if (s != 0) {
                uint64_t m = uabs64(v);
                uint64_t q = m / s, r = m % s; /* s is a power of two: shift and mask */
                uint64_t mag = q + (2 * r >= s);
                if (mag > 127) return AHO_ERR_FIXED_OVERFLOW;
                code = v < 0 ? -(int)mag : (int)mag;
            }
            codes[base + l] = (int8_t)code;
        }
    }
    if (!dequantizes(codes, scales, n)) return AHO_ERR_FIXED_OVERFLOW;
    return AHO_OK;
}

int aho_quant_act_f32(const float *x, size_t n, int8_t *codes, int64_t *scales) {
    int64_t *q = (int64_t *)malloc((n ? n : 1) * sizeof(int64_t));
    if (!q) return AHO_ERR_LENGTH_OVERFLOW;
    for (size_t i = 0; i < n; i++) {
        uint32_t bits;
        memcpy(&bits, &x[i], 4);
        int st = aho_to_q32(bits, &q[i]);
        if (st) {
            free(q);
            return st;
        }
    }
    int st = aho_quant_act(q, n, codes, scales);
    free(q);
    return st;
}

int aho_dequant_act(const int8_t *codes, const int64_t *scales, size_t n, int64_t *xhat) {
    for (size_t i = 0; i < n; i++)
        if (__builtin_mul_overflow(scales[i / 32], (int64_t)codes[i], &xhat[i]))
            return AHO_ERR_FIXED_OVERFLOW;
    return AHO_OK;
}

/* format/quant.rs:482-491 (ggml get_scale_min_k4). */
static void q4k_scale_min(const uint8_t *s, int j, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* format/quant.rs:574-599: the 256 Q6_K codes in output order, already minus 32. */
static void q6k_codes(const uint8_t *blk, int8_t *out) {
    const uint8_t *ql = blk, *qh = blk + 128;
    for (int n = 0; n < 2; n++)
        for (int l = 0; l < 32; l++) {
            uint8_t hi = qh[32 * n + l];
            out[128 * n + l] = (int8_t)(((ql[64 * n + l] & 0xF) | (((hi >> 0) & 3) << 4)) - 32);
            out[128 * n + l + 32] = (int8_t)(((ql[64 * n + l + 32] & 0xF) | (((hi >> 2) & 3) << 4)) - 32);
            out[128 * n + l + 64] = (int8_t)(((ql[64 * n + l] >> 4) | (((hi >> 4) & 3) << 4)) - 32);
            out[128 * n + l + 96] = (int8_t)(((ql[64 * n + l + 32] >> 4) | (((hi >> 6) & 3) << 4)) - 32);
        }
}

/* format/quant.rs:263-297: the 32 Q5_0 codes in output order, already minus 16.  qs[j]'s low
 * nibble is output j, its high nibble output 16 + j; the fifth bit of output j is bit j of qh read
 * as a little-endian u32, that of output 16 + j is bit 16 + j. */
static void q50_codes(const uint8_t *blk, int8_t *out) {
    const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
    const uint8_t *qs = blk + 6;
    for (int j = 0; j < 16; j++) {
        out[j] = (int8_t)((int)((qs[j] & 0xF) | (((qh >> j) & 1) << 4)) - 16);
        out[16 + j] = (int8_t)((int)((qs[j] >> 4) | (((qh >> (16 + j)) & 1) << 4)) - 16);
    }
}

/* format/quant.rs:336-364 and :426-458: Q2_K / Q3_K codes in output order.  Each half of 128
 * outputs reads its 32 qs bytes four times, one bit pair per pass (shift 0, 2, 4, 6); a pass emits
 * the 16 bytes of plane 0, then the 16 of plane 1.  Q3_K subtracts 4 from each value whose hmask
 * bit is clear: mask byte 16*plane + l, bit (4*half + pass). */
static void k23_codes(const uint8_t *qs, const uint8_t *hm, int8_t *out) {
    int y = 0;
    for (int half = 0; half < 2; half++)
        for (int pass = 0; pass < 4; pass++)
            for (int plane = 0; plane < 2; plane++)
                for (int l = 0; l < 16; l++, y++) {
                    int v = (qs[32 * half + 16 * plane + l] >> (2 * pass)) & 3;
                    if (hm && !((hm[16 * plane + l] >> (4 * half + pass)) & 1)) v -= 4;
                    out[y] = (int8_t)v;
                }
}

/* format/quant.rs:391-417: the sixteen 6-bit Q3_K scales from the 12 packed bytes, as the four
 * little-endian words of kmask shuffles (kmask1 = 0x03030303, kmask2 = 0x0f0f0f0f). */
static void q3k_scales(const uint8_t *p, int *sc) {
    uint32_t a0 = (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
    uint32_t a1 = (uint32_t)p[4] | (uint32_t)p[5] << 8 | (uint32_t)p[6] << 16 | (uint32_t)p[7] << 24;
    uint32_t t = (uint32_t)p[8] | (uint32_t)p[9] << 8 | (uint32_t)p[10] << 16 | (uint32_t)p[11] << 24;
    const uint32_t m1 = 0x03030303u, m2 = 0x0f0f0f0fu;
    uint32_t w[4] = {(a0 & m2) | ((t & m1) << 4), (a1 & m2) | (((t >> 2) & m1) << 4),
                     ((a0 >> 4) & m2) | (((t >> 4) & m1) << 4), ((a1 >> 4) & m2) | (((t >> 6) & m1) << 4)};
    for (int j = 0; j < 16; j++) sc[j] = (int)((w[j / 4] >> (8 * (j % 4))) & 0xff);
}

/* The integer codes of one super-block / block in output order (Q4_K: nibbles 0..15). */
static void q4k_codes(const uint8_t *blk, uint8_t *out) {
    const uint8_t *qs = blk + 16;
    for (int b = 0; b < 4; b++)
        for (int l = 0; l < 32; l++) {
            out[64 * b + l] = qs[32 * b + l] & 0xF;
            out[64 * b + 32 + l] = qs[32 * b + l] >> 4;
        }
}

/* num/dequant.rs:99-122 with the family rows :315-351, :514-617, :619-671.  Every product is
 * exact in int64 for finite scales, so only NonFiniteScale can refuse here. */
int aho_dequant_row(uint32_t t, const uint8_t *row, size_t row_len, size_t n, int64_t *out) {
    size_t qk, bb;
    if (!aho_block_geom(t, &qk, &bb)) return AHO_ERR_UNSUPPORTED_QUANT;
    size_t blocks = (n + qk - 1) / qk;
    if (row_len < blocks * bb) return AHO_ERR_SHORT_PAYLOAD;
    int64_t vals[QK_K];
    for (size_t b = 0; b < blocks; b++) {
        const uint8_t *blk = row + b * bb;
        size_t take = n - b * qk < qk ? n - b * qk : qk;
        int st;
        if (t == AHO_Q8_0) {
            int64_t d;
            if ((st = aho_f16_to_fixed(rd16(blk), &d))) return st;
            for (size_t l = 0; l < take; l++) out[b * qk + l] = d * (int64_t)(int8_t)blk[2 + l];
        } else if (t == AHO_Q5_0) {
            /* num/dequant.rs:353-380: w = d * (q - 16) */
            int64_t d;
            if ((st = aho_f16_to_fixed(rd16(blk), &d))) return st;
            int8_t c[32];
            q50_codes(blk, c);
            for (size_t l = 0; l < take; l++) out[b * qk + l] = d * (int64_t)c[l];
        } else if (t == AHO_Q2_K) {
            /* num/dequant.rs:395-462: w = d*sc*q - dmin*m per 16-group (sc low nibble, m high) */
            int64_t d, dmin;
            if ((st = aho_f16_to_fixed(rd16(blk + 80), &d))) return st;
            if ((st = aho_f16_to_fixed(rd16(blk + 82), &dmin))) return st;
            int8_t c[QK_K];
            k23_codes(blk + 16, NULL, c);
            for (int g = 0; g < 16; g++) {
                int64_t slope = d * (blk[g] & 0xF), icpt = dmin * (blk[g] >> 4);
                for (int l = 0; l < 16; l++) vals[16 * g + l] = slope * c[16 * g + l] - icpt;
            }
            memcpy(out + b * qk, vals, take * sizeof(int64_t));
        } else if (t == AHO_Q3_K) {
            /* num/dequant.rs:464-512: w = d*(sc-32)*c per 16-group */
            int64_t d;
            if ((st = aho_f16_to_fixed(rd16(blk + 108), &d))) return st;
            int8_t c[QK_K];
            int sc[16];
            k23_codes(blk + 32, blk, c);
            q3k_scales(blk + 96, sc);
            for (int g = 0; g < 16; g++) {
                int64_t slope = d * (sc[g] - 32);
                for (int l = 0; l < 16; l++) vals[16 * g + l] = slope * c[16 * g + l];
            }
            memcpy(out + b * qk, vals, take * sizeof(int64_t));
        } else if (t == AHO_Q4_K) {
            int64_t d, dmin;
            if ((st = aho_f16_to_fixed(rd16(blk), &d))) return st;
            if ((st = aho_f16_to_fixed(rd16(blk + 2), &dmin))) return st;
            uint8_t codes[QK_K];
            q4k_codes(blk, codes);
            for (int j = 0; j < 8; j++) {
                int sc, m;
                q4k_scale_min(blk + 4, j, &sc, &m);
                int64_t slope = d * sc, icpt = dmin * m;
                for (int l = 0; l < 32; l++) vals[32 * j + l] = slope * codes[32 * j + l] - icpt;
            }
            memcpy(out + b * qk, vals, take * sizeof(int64_t)); /* push_prefix, dequant.rs:76-83 */
        } else {
            int64_t d;
            if ((st = aho_f16_to_fixed(rd16(blk + 208), &d))) return st;
            int8_t codes[QK_K];
            q6k_codes(blk, codes);
            for (int g = 0; g < 16; g++) {
                int64_t slope = d * (int64_t)(int8_t)blk[192 + g];
                for (int l = 0; l < 16; l++) vals[16 * g + l] = slope * codes[16 * g + l];
            }
            memcpy(out + b * qk, vals, take * sizeof(int64_t));
        }
    }
    return AHO_OK;
}

/* round_shift_32 (num/value.rs:9-12) with the i64 range check of row_dot_fixed. */
static int finish_i64(i128 acc, int64_t *y) {
    i128 r;
    if (__builtin_add_overflow(acc, (i128)1 << 31, &r)) return AHO_ERR_OUTPUT_OVERFLOW;
    r >>= 32;
    if (r > (i128)INT64_MAX || r < (i128)INT64_MIN) return AHO_ERR_OUTPUT_OVERFLOW;
    *y = (int64_t)r;
    return AHO_OK;
}

/* ops/matvec.rs:149-222 (row_dot_fixed :86-117). */
int aho_matvec_fixed(uint32_t t, const uint8_t *raw, size_t raw_len, size_t n_out, size_t n_in,
                     const int64_t *x, size_t x_len, int64_t *y) {
    size_t qk, bb;
    if (!aho_block_geom(t, &qk, &bb)) return AHO_ERR_UNSUPPORTED_QUANT;
    if (x_len != n_in) return AHO_ERR_SHAPE_MISMATCH;
    size_t row_bytes, need;
    if (__builtin_mul_overflow((n_in + qk - 1) / qk, bb, &row_bytes)) return AHO_ERR_LENGTH_OVERFLOW;
    if (__builtin_mul_overflow(n_out, row_bytes, &need)) return AHO_ERR_LENGTH_OVERFLOW;
    if (raw_len < need) return AHO_ERR_SHORT_PAYLOAD;
    int64_t *w = (int64_t *)malloc((n_in ? n_in : 1) * sizeof(int64_t));
    if (!w) return AHO_ERR_LENGTH_OVERFLOW;
    int st = AHO_OK;
    for (size_t o = 0; o < n_out && st == AHO_OK; o++) {
        st = aho_dequant_row(t, raw + o * row_bytes, row_bytes, n_in, w);
        if (st) break;
        i128 acc = 0;
        for (size_t i = 0; i < n_in; i++) {
            i128 p;
            if (__builtin_mul_overflow((i128)w[i], (i128)x[i], &p) ||
                __builtin_add_overflow(acc, p, &acc)) {
                st = AHO_ERR_ACCUMULATOR_OVERFLOW;
                break;
            }
        }
        if (st) break;
        st = finish_i64(acc, &y[o]);
    }
    free(w);
    return st;
}

/* chart/mod.rs:1887-1925: the contract is matvec_fixed on QuantAct::dequant, after the
 * FixedOverflow refusal for an activation with no Q32.32 value. */
int aho_matvec_q8act(uint32_t t, const uint8_t *raw, size_t raw_len, size_t n_out, size_t n_in,
                     const int8_t *codes, const int64_t *scales, size_t n_codes, int64_t *y) {
    int64_t *xhat = (int64_t *)malloc((n_codes ? n_codes : 1) * sizeof(int64_t));
    if (!xhat) return AHO_ERR_LENGTH_OVERFLOW;
    int st = aho_dequant_act(codes, scales, n_codes, xhat);
    if (st == AHO_OK) st = aho_matvec_fixed(t, raw, raw_len, n_out, n_in, xhat, n_codes, y);
    free(xhat);
    return st;
}

int aho_block_dots(uint32_t t, const uint8_t *row, size_t row_len, size_t n_in,
                   const int8_t *codes, int32_t *dots, int32_t *xsums) {
    size_t qk, bb;
    if (!aho_block_geom(t, &qk, &bb)) return AHO_ERR_UNSUPPORTED_QUANT;
    size_t blocks = (n_in + qk - 1) / qk;
    if (row_len < blocks * bb) return AHO_ERR_SHORT_PAYLOAD;
    size_t nb32 = (n_in + 31) / 32;
    for (size_t b = 0; b < nb32; b++) {
        int32_t s = 0;
        for (size_t l = b * 32; l < n_in && l < b * 32 + 32; l++) s += codes[l];
        xsums[b] = s;
    }
    if (t == AHO_Q8_0) {
        for (size_t b = 0; b < nb32; b++) {
            int32_t s = 0;
            for (size_t l = 0; l < 32 && b * 32 + l < n_in; l++)
                s += (int32_t)(int8_t)row[b * 34 + 2 + l] * codes[b * 32 + l];
            dots[b] = s;
        }
    } else if (t == AHO_Q5_0) {
        /* chart/mod.rs:630-712: one group per block, dot = sum (q - 16) * xq */
        for (size_t b = 0; b < nb32; b++) {
            int8_t c[32];
            q50_codes(row + b * Q5_0_BYTES, c);
            int32_t s = 0;
            for (size_t l = 0; l < 32 && b * 32 + l < n_in; l++) s += (int32_t)c[l] * codes[b * 32 + l];
            dots[b] = s;
        }
    } else if (t == AHO_Q4_K) {
        for (size_t sb = 0; sb < blocks; sb++) {
            uint8_t c[QK_K];
            q4k_codes(row + sb * bb, c);
            for (int j = 0; j < 8; j++) {
                size_t g = sb * 8 + j;
                if (g >= nb32) break;
                int32_t s = 0;
                for (int l = 0; l < 32 && g * 32 + l < n_in; l++) s += c[32 * j + l] * codes[g * 32 + l];
                dots[g] = s;
            }
        }
    } else {
        size_t nb16 = (n_in + 15) / 16;
        for (size_t sb = 0; sb < blocks; sb++) {
            int8_t c[QK_K];
            const uint8_t *blk = row + sb * bb;
            if (t == AHO_Q2_K) k23_codes(blk + 16, NULL, c);
            else if (t == AHO_Q3_K) k23_codes(blk + 32, blk, c);
            else q6k_codes(blk, c);
            for (int j = 0; j < 16; j++) {
                size_t g = sb * 16 + j;
                if (g >= nb16) break;
                int32_t s = 0;
                for (int l = 0; l < 16 && g * 16 + l < n_in; l++) s += c[16 * j + l] * codes[g * 16 + l];
                dots[g] = s;
            }
        }
    }
    return AHO_OK;
}

int aho_row_absdot(uint32_t t, const uint8_t *raw, size_t raw_len, size_t n_out, size_t n_in,
                   const int8_t *codes, const int64_t *scales, double *out) {
    size_t row_bytes;
    int st = aho_row_bytes(t, n_in, &row_bytes);
    if (st) return st;
    if (raw_len < n_out * row_bytes) return AHO_ERR_SHORT_PAYLOAD;
    int64_t *w = (int64_t *)malloc((n_in ? n_in : 1) * sizeof(int64_t));
    if (!w) return AHO_ERR_LENGTH_OVERFLOW;
    const double two_m64 = 1.0 / 18446744073709551616.0;
    for (size_t o = 0; o < n_out; o++) {
        st = aho_dequant_row(t, raw + o * row_bytes, row_bytes, n_in, w);
        if (st) break;
        double s = 0.0;
        for (size_t i = 0; i < n_in; i++) {
            double xv = (double)scales[i / 32] * (double)codes[i];
            s += (double)w[i] * (xv < 0 ? -xv : xv) * (w[i] < 0 ? -1.0 : 1.0);
        }
        out[o] = s * two_m64;
    }
    free(w);
    return st;
}
