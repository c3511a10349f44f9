/*
 * ah_oracle_ffn.c -- CPU restatement of the FFN's SwiGLU element, the step between the gate/up
 * projections and the down projection of apeiron's quantized FFN.
 *
 * TEST INFRASTRUCTURE ONLY (see ah_oracle.h).  Exact integer arithmetic in __int128.
 *
 *   aho_fixed_exp   numeric/fixed_exp.rs (exp_reduce :40-66, exp_horner :68-84, exp_scale
 *                   :86-118, fixed_exp :120-131): exp(x) in Q32.32 on [-16, 21]
 *   aho_silu_fixed  engine/ops/silu.rs:18-60: round(|v| * 2^32 / (2^32 + exp(-v))) with v's sign
 *                   on -21 < v < 16 (Q32.32 units), v above, 0 below
 *   aho_swiglu      engine/chart/ffn.rs:246-252 (swiglu_one): round_shift_32(silu(gate) * up)
 */
#include "ah_oracle.h"

#include <stdlib.h>
#include <string.h>

typedef __int128 i128;
#define ONE ((int64_t)1 << 32)
static const int64_t LN2_Q32 = 2977044472LL;        /* round(ln 2 * 2^32)     */
static const int64_t LN2_RECIP_Q32 = 6196328019LL;  /* round(2^32 / ln 2)     */

/* round(v / 2^32), ties away from zero (fixed_exp.rs round_div_2p32) */
static i128 round_div_2p32(i128 v) {
    const i128 half = (i128)1 << 31;
    return v >= 0 ? (v + half) >> 32 : -((-v + half) >> 32);
}

int aho_fixed_exp(int64_t x, int64_t *out) {
    if (x < -16 * ONE || x > 21 * ONE) return AHO_ERR_EXP_RANGE;
    /* k = round(x / ln 2) (ties up), r = x - k ln 2 */
    const i128 shifted = ((i128)x * LN2_RECIP_Q32 + ((i128)1 << 63)) >> 64;
    const int64_t k = (int64_t)shifted;
    const int64_t r = x - k * LN2_Q32;
    /* Taylor terms 1/7! .. 1/0! in Q32.32, Horner from the highest */
    static const int64_t c[8] = {852176, 5965232, 35791394, 178956971, 715827883,
                                 2147483648LL, 4294967296LL, 4294967296LL};
    i128 acc = c[0];
    for (int i = 1; i < 8; ++i) acc = round_div_2p32(acc * r) + c[i];
    if (k >= 0) {
        if (k >= 64) return AHO_ERR_EXP_RANGE;
        const i128 s = acc << k;
        if (s > INT64_MAX || s < INT64_MIN) return AHO_ERR_EXP_RANGE;
        *out = (int64_t)s;
    } else {
        const int64_t n = -k;
        if (n >= 64) {
            *out = 0;
            return AHO_OK;
        }
        const i128 s = (acc + ((i128)1 << (n - 1))) >> n;
        if (s > INT64_MAX || s < INT64_MIN) return AHO_ERR_EXP_RANGE;
        *out = (int64_t)s;
    }
    return AHO_OK;
}

int aho_silu_fixed(int64_t v, int64_t *out) {
    if (v >= 16 * ONE) {
        *out = v;
        return AHO_OK;
    }
    if (v <= -21 * ONE) {
        *out = 0;
        return AHO_OK;
    }
    int64_t e;
    if (aho_fixed_exp(-v, &e)) return AHO_ERR_EXP_RANGE;
    if (e > INT64_MAX - ONE) return AHO_ERR_FFN_OVERFLOW;
    const int64_t den = ONE + e;
    if (den <= 0) return AHO_ERR_ZERO_DENOMINATOR;
    const i128 mag = v < 0 ? -(i128)v : (i128)v;
    const i128 num = mag * ONE;
    const i128 q = (num + den / 2) / den; /* div_round_nearest (num.rs value.rs:5-7), num >= 0 */
    const i128 s = v < 0 ? -q : q;
    if (s > INT64_MAX || s < INT64_MIN) return AHO_ERR_FFN_OVERFLOW;
    *out = (int64_t)s;
    return AHO_OK;
}

int aho_swiglu(int64_t gate, int64_t up, int64_t *h) {
    int64_t s;
    const int st = aho_silu_fixed(gate, &s);
    if (st) return st;
    const i128 prod = (i128)s * up;                      /* |i64 * i64| < 2^127: never overflows */
    const i128 r = (prod + ((i128)1 << 31)) >> 32;       /* round_shift_32 (value.rs:10-12)    */
    if (r > INT64_MAX || r < INT64_MIN) return AHO_ERR_FFN_OVERFLOW;
    *h = (int64_t)r;
    return AHO_OK;
}

/* The FFN's hidden activation from f32 gate/up outputs: each converted exactly (to_q32, num/fp.rs
 * :186-230), SwiGLU'd, then quant_act (chart/mod.rs:258), the input of the down projection.
 * The first refusal in element order wins (conversion before SwiGLU per element); hidden values
 * are written to h (n entries) when h is not NULL. */
int aho_swiglu_quant_f32(const float *gate, const float *up, size_t n, int8_t *codes,
                         int64_t *scales, int64_t *h) {
    int64_t *buf = h ? h : (int64_t *)malloc((n ? n : 1) * sizeof(int64_t));
    if (!buf) return -1;
    int st = AHO_OK;
    for (size_t i = 0; i < n && st == AHO_OK; ++i) {
        uint32_t gb, ub;
        memcpy(&gb, gate + i, 4);
        memcpy(&ub, up + i, 4);
        int64_t g, u;
        st = aho_to_q32(gb, &g);
        if (st == AHO_OK) st = aho_to_q32(ub, &u);
        if (st == AHO_OK) st = aho_swiglu(g, u, &buf[i]);
    }
    if (st == AHO_OK) st = aho_quant_act(buf, n, codes, scales);
    if (!h) free(buf);
    return st;
}
