/*
 * ah_cpu_fast.c -- the reference's fast CPU projection restated for host timing.
 *
 * TEST/BENCH INFRASTRUCTURE ONLY (the CPU baseline leg of bench.py and its tests).
 *
 * Restates the chart row kernels of the reference: each 32-lane group yields an exact i32 dot
 * (chart/x86.rs:175-449; AVX-VNNI vpdpbusd where the host has it, else AVX2 vpmaddubsw/vpmaddwd,
 * chosen at run time as dot32_lanes does, x86.rs:175-205) and one i128 fold
 * acc += S_b * (w_scale*dot - w_min*xsum) (RowAcc::emit, chart/mod.rs:501-514); Q8_0, Q5_0 and Q4_K
 * rows go two at a time, sharing each block's activation loads (tiled2, x86.rs:782-1192); the row
 * ends with round_shift_32 and the i64 range check (chart/mod.rs:1739-1753).  Rows are split into
 * contiguous chunks over a thread pool (chart/ffn.rs:667-727); the GEMM form decodes each pair of
 * rows once and dots them against every token column (chart/kcols.rs k-column form).  The cores
 * live in ah_cpu_rows.inc, compiled once per dot form.
 * When the call-level fast bound (chart/mod.rs:336-383) fails, or a weight scale is
 * non-finite, the call falls back to the exact contract, as the reference does
 * (chart/mod.rs:1847-1854), so the values are always aho_matvec_q8act's.
 */
#include "ah_oracle.h"

#include <cpuid.h>
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

/* ---- lane sums ---------------------------------------------------------------------- */

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

/* Q4_K sub-block scale and min of sub-block j from the 12 packed bytes (format/quant.rs:200-213). */
static inline void q4k_sc_m(const uint8_t *scb, int j, int *scv, int *mv) {
    if (j < 4) {
        *scv = scb[j] & 63;
        *mv = scb[j + 4] & 63;
    } else {
        *scv = (scb[j + 4] & 0xF) | ((scb[j - 4] >> 6) << 4);
        *mv = (scb[j + 4] >> 4) | ((scb[j] >> 6) << 4);
    }
}

/* ---- the x86 cores, once per dot form -------------------------------------------------- */

#define RK_VNNI 0
#define RK_ATTR __attribute__((target("avx2")))
#define RK(name) name##_avx2
#include "ah_cpu_rows.inc"
#undef RK_VNNI
#undef RK_ATTR
#undef RK

#define RK_VNNI 1
#define RK_ATTR __attribute__((target("avx2,avxvnni")))
#define RK(name) name##_vnni
#include "ah_cpu_rows.inc"
#undef RK_VNNI
#undef RK_ATTR
#undef RK

/* The host's cores: AVX-VNNI is CPUID leaf 7, sub-leaf 1, EAX bit 4 (on top of AVX2). */
static int host_path(void) {
    if (!aho_has_avx2()) return AHO_CPU_PORTABLE;
    unsigned a, b, c, d;
    if (__get_cpuid_count(7, 1, &a, &b, &c, &d) && (a & (1u << 4))) return AHO_CPU_VNNI;
    return AHO_CPU_AVX2;
}

static int forced_path = -1;

int aho_set_cpu_path(int path) {
    int host = host_path();
    forced_path = path < 0 ? -1 : path > host ? host : path;
    return aho_cpu_path();
}

int aho_cpu_path(void) { return forced_path >= 0 ? forced_path : host_path(); }

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
    const int path = aho_cpu_path();
    if (n_threads < 1) n_threads = 1;
    /* tasks = max(chunks, 2*width) contiguous row chunks (chart/ffn.rs:705-706). */
    size_t tasks = (size_t)(2 * n_threads);
    if (tasks > n_out) tasks = n_out ? n_out : 1;
    size_t per = n_out ? (n_out + tasks - 1) / tasks : 0;
    int nonfinite = 0, overflow = 0;
#pragma omp parallel for schedule(static) num_threads(n_threads) reduction(| : nonfinite, overflow)
    for (size_t task = 0; task < tasks; task++) {
        size_t lo = task * per, hi = lo + per < n_out ? lo + per : n_out;
        /* two decode buffers (rows r and r + 1) for the decoded forms */
        int8_t *wc = (int8_t *)malloc(2 * (nb32 * 32 + 32));
        grp_coef *cf = (grp_coef *)malloc(2 * (nb32 + 8) * sizeof(grp_coef));
        if (path == AHO_CPU_VNNI) {
            rows_task_vnni(t, raw, row_bytes, lo, hi, nb32, &pa, scales, wc, cf, y, &nonfinite, &overflow);
        } else if (path == AHO_CPU_AVX2) {
            rows_task_avx2(t, raw, row_bytes, lo, hi, nb32, &pa, scales, wc, cf, y, &nonfinite, &overflow);
        } else {
            for (size_t r = lo; r < hi; r++) {
                if (decode_row(t, raw + r * row_bytes, nb32, wc, cf)) {
                    nonfinite = 1;
                    break;
                }
                if (finish(row_acc_portable(wc, cf, nb32, pa.codes, scales, pa.xs32), &y[r])) overflow = 1;
            }
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
    /* matmat_q8act routing (kern/matmat.rs:140-180): the K-quant k-column kernels admit only
     * whole super-blocks (K % 256 == 0, chart/kcols.rs:1399-1518); other K-quant widths take the
     * per-column matvec_q8act path (matmat.rs:392-413), one projection per token column, in order. */
    if ((t == AHO_Q4_K || t == AHO_Q6_K) && n_in % 256 != 0) {
        for (size_t c = 0; c < n_tok; c++) {
            int st = aho_matvec_q8act_fast(t, raw, raw_len, n_out, n_in, codes + c * n_in, scales + c * nb32,
                                           y + c * n_out, n_threads);
            if (st) return st;
        }
        return AHO_OK;
    }
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
    const int path = aho_cpu_path();
    int nonfinite = 0, overflow = 0;
    if (ret == AHO_OK) {
        if (n_threads < 1) n_threads = 1;
        const size_t pairs = (n_out + 1) / 2;
#pragma omp parallel num_threads(n_threads) reduction(| : nonfinite, overflow)
        {
            int8_t *wc = (int8_t *)malloc(2 * (nb32 * 32 + 32));
            grp_coef *cf = (grp_coef *)malloc(2 * (nb32 + 8) * sizeof(grp_coef));
#pragma omp for schedule(static)
            for (size_t p = 0; p < pairs; p++) {
                const size_t r0 = 2 * p, r1 = r0 + 2 < n_out ? r0 + 2 : n_out;
                if (path == AHO_CPU_VNNI) {
                    gemm_rows_vnni(t, raw, row_bytes, r0, r1, nb32, n_out, n_tok, pas, slow, scales, wc, cf, y,
                                   &nonfinite, &overflow);
                } else if (path == AHO_CPU_AVX2) {
                    gemm_rows_avx2(t, raw, row_bytes, r0, r1, nb32, n_out, n_tok, pas, slow, scales, wc, cf, y,
                                   &nonfinite, &overflow);
                } else {
                    for (size_t r = r0; r < r1; r++) {
                        if (decode_row(t, raw + r * row_bytes, nb32, wc, cf)) {
                            nonfinite = 1;
                            continue;
                        }
                        for (size_t c = 0; c < n_tok; c++) {
                            if (slow[c]) continue;
                            i128 acc = row_acc_portable(wc, cf, nb32, pas[c].codes, scales + c * nb32, pas[c].xs32);
                            if (finish(acc, &y[c * n_out + r])) overflow = 1;
                        }
                    }
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
