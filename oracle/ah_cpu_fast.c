/*
 * ah_cpu_fast.c -- the reference's fast CPU projection restated for host timing.
 *
 * TEST/BENCH INFRASTRUCTURE ONLY (the CPU baseline leg of bench.py and its tests).
 *
 * Restates the chart row kernels of the reference, one row at a time (the reference's two-row
 * tiling, x86.rs:782-1192, and AVX-VNNI cores, x86.rs:74-85, are not restated: this is a lower
 * bound on its rate): each 32-lane group yields an exact i32
 * dot (AVX2 maddubs/madd, chart/x86.rs:175-449) and one i128 fold
 * acc += S_b * (w_scale*dot - w_min*xsum) (RowAcc::emit, chart/mod.rs:501-514); the row ends
 * with round_shift_32 and the i64 range check (chart/mod.rs:1739-1753).  Rows are split into
 * contiguous chunks over a thread pool (chart/ffn.rs:667-727); the GEMM form decodes each
 * row's groups once and dots them against every token column (chart/kcols.rs k-column form).
 * When the call-level fast bound (chart/mod.rs:336-383) fails, or a weight scale is
 * non-finite, the call falls back to the exact contract, as the reference does
 * (chart/mod.rs:1847-1854), so the values are always aho_matvec_q8act's.
 */
#include "ah_oracle.h"

#include <immintrin.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

typedef __int128 i128;

int aho_has_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") ? 1 : 0;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* f16 -> Q32.32, with bit 0 set as the non-finite marker (finite values are multiples of 2^8). */
static inline int64_t f16_fixed_or_marker(uint16_t h) {
    int64_t v;
    return aho_f16_to_fixed(h, &v) ? 1 : v;
}

/* ---- exact 32-lane dots -------------------------------------------------------------- */

__attribute__((target("avx2"))) static inline __m256i dot_i8_avx2(__m256i w, __m256i x) {
    /* |w| as u8 times x*sign(w): maddubs pairs stay below 2*128*127 = 32512 (no saturation). */
    const __m256i ones = _mm256_set1_epi16(1);
    __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(x, w));
    return _mm256_madd_epi16(p, ones);
}

__attribute__((target("avx2"))) static inline __m256i dot_u8_avx2(__m256i u, __m256i x) {
    const __m256i ones = _mm256_set1_epi16(1);
    return _mm256_madd_epi16(_mm256_maddubs_epi16(u, x), ones);
}

__attribute__((target("avx2"))) static inline int32_t hsum8(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
    return _mm_cvtsi128_si32(s);
}

/* Sum of the first four / last four i32 lanes (the two 16-lane halves of a 32-lane dot). */
__attribute__((target("avx2"))) static inline void hsum_halves(__m256i v, int32_t *lo, int32_t *hi) {
    __m128i a = _mm256_castsi256_si128(v), b = _mm256_extracti128_si256(v, 1);
    a = _mm_add_epi32(a, _mm_shuffle_epi32(a, 0x4e));
    a = _mm_add_epi32(a, _mm_shuffle_epi32(a, 0xb1));
    b = _mm_add_epi32(b, _mm_shuffle_epi32(b, 0x4e));
    b = _mm_add_epi32(b, _mm_shuffle_epi32(b, 0xb1));
    *lo = _mm_cvtsi128_si32(a);
    *hi = _mm_cvtsi128_si32(b);
}

/* ---- per-row decoded form -------------------------------------------------------------- */

/* One 32-lane group of a decoded row: codes (Q8_0 i8, Q4_K nibble, Q6_K u-32) and the
 * exact coefficients of term = clo*Dlo + chi*Dhi - cmin*X (Dlo/Dhi: the two 16-lane halves). */
typedef struct {
    int64_t clo, chi, cmin;
} grp_coef;

/* Decode one row into K_pad codes and per-32 coefficients.  Returns 1 on a non-finite scale. */
static int decode_row(uint32_t t, const uint8_t *row, size_t nb32, int8_t *codes, grp_coef *cf) {
    int64_t bad = 0;
    if (t == AHO_Q8_0) {
        for (size_t b = 0; b < nb32; b++) {
            const uint8_t *blk = row + 34 * b;
            int64_t d = f16_fixed_or_marker(rd16(blk));
            bad |= d;
            cf[b].clo = cf[b].chi = d;
            cf[b].cmin = 0;
            memcpy(codes + 32 * b, blk + 2, 32);
        }
    } else if (t == AHO_Q5_0) {
        /* format/quant.rs:263-297 (the five-bit codes minus 16) */
        for (size_t b = 0; b < nb32; b++) {
            const uint8_t *blk = row + 22 * b;
            int64_t d = f16_fixed_or_marker(rd16(blk));
            bad |= d;
            cf[b].clo = cf[b].chi = d;
            cf[b].cmin = 0;
            const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                                ((uint32_t)blk[5] << 24);
            for (int j = 0; j < 16; j++) {
                codes[32 * b + j] = (int8_t)((int)((blk[6 + j] & 0xF) | (((qh >> j) & 1) << 4)) - 16);
                codes[32 * b + 16 + j] = (int8_t)((int)((blk[6 + j] >> 4) | (((qh >> (16 + j)) & 1) << 4)) - 16);
            }
        }
    } else if (t == AHO_Q4_K) {
        size_t nsb = (nb32 + 7) / 8;
        for (size_t s = 0; s < nsb; s++) {
            const uint8_t *blk = row + 144 * s;
            int64_t d = f16_fixed_or_marker(rd16(blk)), dm = f16_fixed_or_marker(rd16(blk + 2));
            bad |= d | dm;
            const uint8_t *sc = blk + 4, *qs = blk + 16;
            for (int j = 0; j < 8 && s * 8 + j < nb32; j++) {
                int scv, mv;
                if (j < 4) {
                    scv = sc[j] & 63;
                    mv = sc[j + 4] & 63;
                } else {
                    scv = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
                    mv = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
                }
                grp_coef *c = &cf[s * 8 + j];
                c->clo = c->chi = d * scv;
                c->cmin = dm * mv;
                for (int l = 0; l < 32; l++)
                    codes[(s * 8 + j) * 32 + l] = (int8_t)((j & 1) ? (qs[32 * (j / 2) + l] >> 4)
                                                                    : (qs[32 * (j / 2) + l] & 0xF));
            }
        }
    } else {
        size_t nsb = (nb32 + 7) / 8;
        for (size_t s = 0; s < nsb; s++) {
            const uint8_t *blk = row + 210 * s;
            int64_t d = f16_fixed_or_marker(rd16(blk + 208));
            bad |= d;
            const uint8_t *ql = blk, *qh = blk + 128;
            int8_t c256[256];
            for (int n = 0; n < 2; n++)
                for (int l = 0; l < 32; l++) {
                    uint8_t hi = qh[32 * n + l];
                    c256[128 * n + l] = (int8_t)(((ql[64 * n + l] & 0xF) | ((hi & 3) << 4)) - 32);
                    c256[128 * n + l + 32] = (int8_t)(((ql[64 * n + l + 32] & 0xF) | (((hi >> 2) & 3) << 4)) - 32);
                    c256[128 * n + l + 64] = (int8_t)(((ql[64 * n + l] >> 4) | (((hi >> 4) & 3) << 4)) - 32);
                    c256[128 * n + l + 96] = (int8_t)(((ql[64 * n + l + 32] >> 4) | (((hi >> 6) & 3) << 4)) - 32);
                }
            for (int j = 0; j < 8 && s * 8 + j < nb32; j++) {
                grp_coef *c = &cf[s * 8 + j];
                c->clo = d * (int64_t)(int8_t)blk[192 + 2 * j];
                c->chi = d * (int64_t)(int8_t)blk[192 + 2 * j + 1];
                c->cmin = 0;
                memcpy(codes + (s * 8 + j) * 32, c256 + 32 * j, 32);
            }
        }
    }
    return (bad & 1) != 0;
}

/* The call-level fast bound, chart/mod.rs:336-383 (narrow form for Q8_0 and Q5_0). */
static int fast_bound_ok(uint32_t t, size_t n_in, const int64_t *scales, size_t nb32) {
    i128 top = t == AHO_Q8_0 ? 128 : t == AHO_Q5_0 ? 16 : t == AHO_Q4_K ? 1008 : 4096;
    i128 smax = 0;
    for (size_t b = 0; b < nb32; b++) {
        i128 a = scales[b] < 0 ? -(i128)scales[b] : (i128)scales[b];
        if (a > smax) smax = a;
    }
    const i128 imax = (i128)(((unsigned __int128)1 << 127) - 1);
    if (t == AHO_Q8_0 || t == AHO_Q5_0) {
        i128 p;
        if (__builtin_mul_overflow(smax, 32 * top * 127, &p) || p > (i128)INT64_MAX) return 0;
    }
    i128 bound = (i128)n_in, f16max = (i128)65504 << 32;
    if (__builtin_mul_overflow(bound, f16max, &bound)) return 0;
    if (__builtin_mul_overflow(bound, top, &bound)) return 0;
    if (__builtin_mul_overflow(bound, (i128)127, &bound)) return 0;
    if (__builtin_mul_overflow(bound, smax, &bound)) return 0;
    return bound < imax;
}

static inline int finish(i128 acc, int64_t *y) {
    i128 r = (acc + ((i128)1 << 31)) >> 32;
    if (r > (i128)INT64_MAX || r < (i128)INT64_MIN) return AHO_ERR_OUTPUT_OVERFLOW;
    *y = (int64_t)r;
    return AHO_OK;
}

/* Exact row accumulator over decoded groups against one token's padded codes. */
__attribute__((target("avx2"))) static i128 row_acc_avx2(const int8_t *wc, const grp_coef *cf,
                                                         size_t nb32, const int8_t *xc,
                                                         const int64_t *sc, const int32_t *xs) {
    i128 acc = 0;
    for (size_t b = 0; b < nb32; b++) {
        __m256i w = _mm256_loadu_si256((const __m256i *)(wc + 32 * b));
        __m256i x = _mm256_loadu_si256((const __m256i *)(xc + 32 * b));
        __m256i p = dot_i8_avx2(w, x);
        int32_t lo, hi;
        hsum_halves(p, &lo, &hi);
        i128 inner = (i128)cf[b].clo * lo + (i128)cf[b].chi * hi - (i128)cf[b].cmin * xs[b];
        acc += (i128)sc[b] * inner;
    }
    return acc;
}

static i128 row_acc_portable(const int8_t *wc, const grp_coef *cf, size_t nb32,
                             const int8_t *xc, const int64_t *sc, const int32_t *xs) {
    i128 acc = 0;
    for (size_t b = 0; b < nb32; b++) {
        int32_t lo = 0, hi = 0;
        for (int l = 0; l < 16; l++) lo += wc[32 * b + l] * xc[32 * b + l];
        for (int l = 16; l < 32; l++) hi += wc[32 * b + l] * xc[32 * b + l];
        i128 inner = (i128)cf[b].clo * lo + (i128)cf[b].chi * hi - (i128)cf[b].cmin * xs[b];
        acc += (i128)sc[b] * inner;
    }
    return acc;
}

/* Direct Q8_0 fast row from the GGUF bytes (no decode pass): the memory-bound decode path. */
__attribute__((target("avx2"))) static int q8_0_row_direct(const uint8_t *row, size_t nb32,
                                                           const int8_t *xc, const int64_t *sc,
                                                           i128 *out) {
    i128 acc = 0;
    int64_t bad = 0;
    for (size_t b = 0; b < nb32; b++) {
        const uint8_t *blk = row + 34 * b;
        int64_t d = f16_fixed_or_marker(rd16(blk));
        bad |= d;
        __m256i w = _mm256_loadu_si256((const __m256i *)(blk + 2));
        __m256i x = _mm256_loadu_si256((const __m256i *)(xc + 32 * b));
        int32_t D = hsum8(dot_i8_avx2(w, x));
        acc += (i128)sc[b] * ((i128)d * D);
    }
    *out = acc;
    return (bad & 1) != 0;
}

/* Direct Q4_K fast row: nibble unpack in registers, chart/x86.rs:386-435 shape. */
__attribute__((target("avx2"))) static int q4_k_row_direct(const uint8_t *row, size_t nb32,
                                                           const int8_t *xc, const int64_t *sc,
                                                           const int32_t *xs, i128 *out) {
    i128 acc = 0;
    int64_t bad = 0;
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    size_t nsb = (nb32 + 7) / 8;
    for (size_t s = 0; s < nsb; s++) {
        const uint8_t *blk = row + 144 * s;
        int64_t d = f16_fixed_or_marker(rd16(blk)), dm = f16_fixed_or_marker(rd16(blk + 2));
        bad |= d | dm;
        const uint8_t *scb = blk + 4;
        for (int p = 0; p < 4; p++) {
            size_t g = s * 8 + 2 * p;
            if (g >= nb32) break;
            __m256i q = _mm256_loadu_si256((const __m256i *)(blk + 16 + 32 * p));
            __m256i lo = _mm256_and_si256(q, m4), hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            int32_t Dl = hsum8(dot_u8_avx2(lo, _mm256_loadu_si256((const __m256i *)(xc + 32 * g))));
            int32_t Dh = hsum8(dot_u8_avx2(hi, _mm256_loadu_si256((const __m256i *)(xc + 32 * g + 32))));
            for (int h = 0; h < 2; h++) {
                int j = 2 * p + h, scv, mv;
                if (j < 4) {
                    scv = scb[j] & 63;
                    mv = scb[j + 4] & 63;
                } else {
                    scv = (scb[j + 4] & 0xF) | ((scb[j - 4] >> 6) << 4);
                    mv = (scb[j + 4] >> 4) | ((scb[j] >> 6) << 4);
                }
                if (g + h >= nb32) break;
                i128 inner = (i128)(d * scv) * (h ? Dh : Dl) - (i128)(dm * mv) * xs[g + h];
                acc += (i128)sc[g + h] * inner;
            }
        }
    }
    *out = acc;
    return (bad & 1) != 0;
}

/* Direct Q6_K fast row: 4+2-bit plane assembly in registers, chart/x86.rs:700-762 shape. */
__attribute__((target("avx2"))) static int q6_k_row_direct(const uint8_t *row, size_t nb32,
                                                           const int8_t *xc, const int64_t *sc,
                                                           const int32_t *xs16, i128 *out) {
    i128 acc = 0;
    int64_t bad = 0;
    const __m256i m4 = _mm256_set1_epi8(0x0F), m2 = _mm256_set1_epi8(0x03);
    size_t nsb = (nb32 + 7) / 8;
    for (size_t s = 0; s < nsb; s++) {
        const uint8_t *blk = row + 210 * s;
        int64_t d = f16_fixed_or_marker(rd16(blk + 208));
        bad |= d;
        for (int n = 0; n < 2; n++) {
            __m256i l0 = _mm256_loadu_si256((const __m256i *)(blk + 64 * n));
            __m256i l1 = _mm256_loadu_si256((const __m256i *)(blk + 64 * n + 32));
            __m256i h = _mm256_loadu_si256((const __m256i *)(blk + 128 + 32 * n));
            __m256i u[4];
            u[0] = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(h, m2), 4));
            u[1] = _mm256_or_si256(_mm256_and_si256(l1, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 2), m2), 4));
            u[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 4), m2), 4));
            u[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(h, 6), m2), 4));
            for (int tq = 0; tq < 4; tq++) {
                size_t g = s * 8 + 4 * n + tq;
                if (g >= nb32) break;
                __m256i x = _mm256_loadu_si256((const __m256i *)(xc + 32 * g));
                int32_t lo, hi;
                hsum_halves(dot_u8_avx2(u[tq], x), &lo, &hi);
                lo -= 32 * xs16[2 * g];
                hi -= 32 * xs16[2 * g + 1];
                const uint8_t *scb = blk + 192 + 8 * n + 2 * tq;
                i128 inner = (i128)(d * (int64_t)(int8_t)scb[0]) * lo + (i128)(d * (int64_t)(int8_t)scb[1]) * hi;
                acc += (i128)sc[g] * inner;
            }
        }
    }
    *out = acc;
    return (bad & 1) != 0;
}

/* Shared per-token activation data: codes padded to whole super-blocks, per-32 and per-16 sums. */
typedef struct {
    int8_t *codes;
    int32_t *xs32, *xs16;
} padded_act;

static int pad_act(const int8_t *codes, size_t n_in, size_t nb32, padded_act *pa) {
    size_t npad = ((nb32 + 7) / 8) * 256 + 32;
    pa->codes = (int8_t *)calloc(npad, 1);
    pa->xs32 = (int32_t *)calloc(nb32 + 8, sizeof(int32_t));
    pa->xs16 = (int32_t *)calloc(2 * nb32 + 16, sizeof(int32_t));
    if (!pa->codes || !pa->xs32 || !pa->xs16) return 1;
    memcpy(pa->codes, codes, n_in);
    for (size_t g = 0; g < 2 * nb32; g++) {
        int32_t s = 0;
        for (int l = 0; l < 16; l++) s += pa->codes[16 * g + l];
        pa->xs16[g] = s;
    }
    for (size_t b = 0; b < nb32; b++) pa->xs32[b] = pa->xs16[2 * b] + pa->xs16[2 * b + 1];
    return 0;
}

static void free_act(padded_act *pa) {
    free(pa->codes);
    free(pa->xs32);
    free(pa->xs16);
}

int aho_matvec_q8act_fast(uint32_t t, const uint8_t *raw, size_t raw_len, size_t n_out,
                          size_t n_in, const int8_t *codes, const int64_t *scales, int64_t *y,
                          int n_threads) {
    size_t row_bytes;
    int st = aho_row_bytes(t, n_in, &row_bytes);
    if (st) return st;
    if (raw_len < n_out * row_bytes) return AHO_ERR_SHORT_PAYLOAD;
    size_t nb32 = (n_in + 31) / 32;
    /* The activation must have a Q32.32 value (the reference's first refusal). */
    for (size_t i = 0; i < n_in; i++) {
        int64_t v;
        if (__builtin_mul_overflow(scales[i / 32], (int64_t)codes[i], &v)) return AHO_ERR_FIXED_OVERFLOW;
    }
    if (!fast_bound_ok(t, n_in, scales, nb32))
        return aho_matvec_q8act(t, raw, raw_len, n_out, n_in, codes, scales, n_in, y);
    padded_act pa;
    if (pad_act(codes, n_in, nb32, &pa)) {
        free_act(&pa);
        return AHO_ERR_LENGTH_OVERFLOW;
    }
    int avx2 = aho_has_avx2();
    if (n_threads < 1) n_threads = 1;
    /* tasks = max(chunks, 2*width) contiguous row chunks (chart/ffn.rs:705-706). */
    size_t tasks = (size_t)(2 * n_threads);
    if (tasks > n_out) tasks = n_out ? n_out : 1;
    size_t per = n_out ? (n_out + tasks - 1) / tasks : 0;
    int nonfinite = 0, overflow = 0;
#pragma omp parallel for schedule(static) num_threads(n_threads) reduction(| : nonfinite, overflow)
    for (size_t task = 0; task < tasks; task++) {
        size_t lo = task * per, hi = lo + per < n_out ? lo + per : n_out;
        int8_t *wc = NULL;
        grp_coef *cf = NULL;
        if (!avx2 || t == AHO_Q5_0) {
            wc = (int8_t *)malloc(nb32 * 32 + 32);
            cf = (grp_coef *)malloc((nb32 + 8) * sizeof(grp_coef));
        }
        for (size_t r = lo; r < hi; r++) {
            const uint8_t *row = raw + r * row_bytes;
            i128 acc = 0;
            int bad;
            if (avx2 && t == AHO_Q5_0) {  /* decoded row, then the shared AVX2 accumulator */
                bad = decode_row(t, row, nb32, wc, cf);
                if (!bad) acc = row_acc_avx2(wc, cf, nb32, pa.codes, scales, pa.xs32);
            } else if (avx2) {
                if (t == AHO_Q8_0) bad = q8_0_row_direct(row, nb32, pa.codes, scales, &acc);
                else if (t == AHO_Q4_K) bad = q4_k_row_direct(row, nb32, pa.codes, scales, pa.xs32, &acc);
                else bad = q6_k_row_direct(row, nb32, pa.codes, scales, pa.xs16, &acc);
            } else {
                bad = decode_row(t, row, nb32, wc, cf);
                if (!bad) acc = row_acc_portable(wc, cf, nb32, pa.codes, scales, pa.xs32);
            }
            if (bad) {
                nonfinite = 1;
                break;
            }
            if (finish(acc, &y[r])) overflow = 1;
        }
        free(wc);
        free(cf);
    }
    free_act(&pa);
    if (nonfinite) return aho_matvec_q8act(t, raw, raw_len, n_out, n_in, codes, scales, n_in, y);
    if (overflow) return AHO_ERR_OUTPUT_OVERFLOW;
    return AHO_OK;
}

int aho_matmat_q8act_fast(uint32_t t, const uint8_t *raw, size_t raw_len, size_t n_out,
                          size_t n_in, size_t n_tok, const int8_t *codes, const int64_t *scales,
                          int64_t *y, int n_threads) {
    size_t row_bytes;
    int st = aho_row_bytes(t, n_in, &row_bytes);
    if (st) return st;
    if (raw_len < n_out * row_bytes) return AHO_ERR_SHORT_PAYLOAD;
    size_t nb32 = (n_in + 31) / 32;
    if (n_tok == 0 || n_out == 0) return AHO_OK;
    /* Per-token admission: a token whose bound fails (or that does not dequantize) takes the
     * per-column contract, as kern/matmat.rs falls back per call. */
    padded_act *pas = (padded_act *)calloc(n_tok, sizeof(padded_act));
    uint8_t *slow = (uint8_t *)calloc(n_tok, 1);
    int ret = AHO_OK;
    for (size_t c = 0; c < n_tok; c++) {
        const int8_t *cc = codes + c * n_in;
        const int64_t *ss = scales + c * nb32;
        int ok = 1;
        for (size_t i = 0; i < n_in && ok; i++) {
            int64_t v;
            if (__builtin_mul_overflow(ss[i / 32], (int64_t)cc[i], &v)) ok = 0;
        }
        if (!ok) {
            ret = AHO_ERR_FIXED_OVERFLOW;
            break;
        }
        if (!fast_bound_ok(t, n_in, ss, nb32)) slow[c] = 1;
        if (pad_act(cc, n_in, nb32, &pas[c])) ret = AHO_ERR_LENGTH_OVERFLOW;
    }
    int avx2 = aho_has_avx2();
    int nonfinite = 0, overflow = 0;
    if (ret == AHO_OK) {
        if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads) reduction(| : nonfinite, overflow)
        {
            int8_t *wc = (int8_t *)malloc(nb32 * 32 + 32);
            grp_coef *cf = (grp_coef *)malloc((nb32 + 8) * sizeof(grp_coef));
#pragma omp for schedule(static)
            for (size_t r = 0; r < n_out; r++) {
                if (decode_row(t, raw + r * row_bytes, nb32, wc, cf)) {
                    nonfinite = 1;
                    continue;
                }
                for (size_t c = 0; c < n_tok; c++) {
                    if (slow[c]) continue;
                    i128 acc = avx2 ? row_acc_avx2(wc, cf, nb32, pas[c].codes, scales + c * nb32, pas[c].xs32)
                                    : row_acc_portable(wc, cf, nb32, pas[c].codes, scales + c * nb32, pas[c].xs32);
                    if (finish(acc, &y[c * n_out + r])) overflow = 1;
                }
            }
            free(wc);
            free(cf);
        }
        if (nonfinite) {
            ret = AHO_ERR_NONFINITE_SCALE;
        } else {
            for (size_t c = 0; c < n_tok && ret == AHO_OK; c++)
                if (slow[c])
                    ret = aho_matvec_q8act(t, raw, raw_len, n_out, n_in, codes + c * n_in,
                                           scales + c * nb32, n_in, y + c * n_out);
            if (ret == AHO_OK && overflow) ret = AHO_ERR_OUTPUT_OVERFLOW;
        }
    }
    for (size_t c = 0; c < n_tok; c++) free_act(&pas[c]);
    free(pas);
    free(slow);
    return ret;
}
