// ah_swiglu.h -- the exact SwiGLU of the fused FFN and the hidden activation's quantizer, shared
// by the decode (N = 1) kernels and the prefill GEMM's fused epilogue.
//
// h = round_shift_32(silu_fixed(to_q32(gate)) * to_q32(up)) (engine/ops/ffn.rs:80,
// engine/ops/silu.rs:18-60, chart/ffn.rs:246-252) in exact integer arithmetic, then quant_act of
// each 32-element block of h (chart/mod.rs:258-334).
#pragma once

#include "ah_internal.h"

namespace {

typedef __int128 i128;
constexpr int64_t kOneQ32 = (int64_t)1 << 32;

// round(v / 2^32), ties away from zero, for |v| <= 2^63 - 2^31, branch-free in i64
AH_DEV int64_t round_div_2p32_i64(int64_t v) {
    const int64_t s = v >> 63;
    const uint64_t a = (uint64_t)((v ^ s) - s);
    const int64_t q = (int64_t)((a + (1ull << 31)) >> 32);
    return (q ^ s) - s;
}
// exp(x) in Q32.32 for x in [-16, 21] (numeric/fixed_exp.rs:40-131): k = round(x / ln 2),
// r = x - k ln 2, the degree-7 Taylor sum of exp(r) by Horner with round_div_2p32, then 2^k.
// The reference sums in i128; here in i64, exactly: |r| <= ln 2 / 2 * 2^32 < 2^30.5 and every
// partial sum lies in (0, e^(ln 2 / 2) * 2^32) < 2^32.6, so each product acc * r stays below
// 2^63 (the bounds are checked step by step against the oracle in the CPU tests).
AH_DEV int fx_exp(int64_t x, int64_t &out) {
    if (x < -16 * kOneQ32 || x > 21 * kOneQ32) return AH_ERR_EXP_RANGE;
    const int64_t k = (int64_t)(((i128)x * 6196328019LL + ((i128)1 << 63)) >> 64);
    const int64_t r = x - k * 2977044472LL;
    int64_t acc = 852176;
    acc = round_div_2p32_i64(acc * r) + 5965232;
    acc = round_div_2p32_i64(acc * r) + 35791394;
    acc = round_div_2p32_i64(acc * r) + 178956971;
    acc = round_div_2p32_i64(acc * r) + 715827883;
    acc = round_div_2p32_i64(acc * r) + 2147483648LL;
    acc = round_div_2p32_i64(acc * r) + 4294967296LL;
    acc = round_div_2p32_i64(acc * r) + 4294967296LL;
    if (k >= 0) {
        // acc * 2^k must be an i64 (the reference's range check on the i128 value)
        if (k >= 63 || acc > (INT64_MAX >> k) || acc < (INT64_MIN >> k)) return AH_ERR_EXP_RANGE;
        out = acc << k;
        return 0;
    }
    const int64_t n = -k;
    if (n >= 63) {
        out = 0;
        return 0;
    }
    out = (acc + ((int64_t)1 << (n - 1))) >> n;
    return 0;
}
// silu(v) = round(|v| * 2^32 / (2^32 + exp(-v))) with v's sign on -21 < v < 16, v above, 0 below
// (engine/ops/silu.rs:18-60).  The quotient is below 2^37: a double estimate of the i128 division,
// then exact correction against the remainder (the hardware has no i128 divide).  The estimate's
// relative error is below 2^-51 (the numerator's and denominator's conversions and the division,
// each within half an ulp), so it is within 2^-14 of the true quotient and its truncation is the
// floor or one off it either way: one correction step makes it exact.
AH_DEV int silu_fx(int64_t v, int64_t &out) {
    if (v >= 16 * kOneQ32) {
        out = v;
        return 0;
    }
    if (v <= -21 * kOneQ32) {
        out = 0;
        return 0;
    }
    int64_t e;
    if (fx_exp(-v, e)) return AH_ERR_EXP_RANGE;
    if (e > INT64_MAX - kOneQ32) return AH_ERR_FFN_OVERFLOW;
    const int64_t den = kOneQ32 + e;
    if (den <= 0) return AH_ERR_ZERO_DENOMINATOR;
    const uint64_t mag = v < 0 ? 0ull - (uint64_t)v : (uint64_t)v;
    const i128 n2 = (i128)mag * kOneQ32 + (den >> 1);  // div_round_nearest's num + den / 2
    const double nd = (double)(uint64_t)(n2 >> 32) * 4294967296.0 + (double)(uint64_t)(n2 & 0xFFFFFFFFu);
    int64_t q = (int64_t)(nd / (double)den);
    const i128 rem = n2 - (i128)q * den;
    q += rem < 0 ? -1 : rem >= den ? 1 : 0;
    out = v < 0 ? -q : q;
    return 0;
}
// h = round_shift_32(silu(gate) * up) (engine/chart/ffn.rs:246-252)
AH_DEV int swiglu_fx(int64_t g, int64_t u, int64_t &h) {
    int64_t s;
    const int st = silu_fx(g, s);
    if (st) return st;
    const i128 r = ((i128)s * u + ((i128)1 << 31)) >> 32;
    if (r > (i128)INT64_MAX || r < (i128)INT64_MIN) return AH_ERR_FFN_OVERFLOW;
    h = (int64_t)r;
    return 0;
}

// Largest value over each aligned group of 32 lanes (every lane of the group gets it): DPP within
// a row of 16 (quad exchanges, then the half-row and row mirrors), then one exchange of rows.
template <int CTRL>
AH_DEV int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false); }
AH_DEV int max32(int v) {
    v = __builtin_elementwise_max(v, dpp_i<0xB1>(v));   // lane ^ 1
    v = __builtin_elementwise_max(v, dpp_i<0x4E>(v));   // lane ^ 2
    v = __builtin_elementwise_max(v, dpp_i<0x141>(v));  // row_half_mirror
    v = __builtin_elementwise_max(v, dpp_i<0x140>(v));  // row_mirror
    return __builtin_elementwise_max(v, __shfl_xor(v, 16, 64));
}

// One hidden element per lane, 32 lanes per hidden block (aligned half-waves; every lane of the
// wave takes part, dead lanes with live = false): the lane converts its gate and up values (f32
// bits) to Q32.32 and forms h = swiglu, then the block is quantized together.  act_scale is
// monotone in the block's largest magnitude, so the block exponent is the largest of the lanes'
// own exponents (a 32-lane max of small integers) and each lane forms its own code.
struct HiddenQ {
    int code;        // the lane's hidden code (0 for a dead lane and for a refused block)
    uint64_t scale;  // the block's scale 2^e (0 for an all-zero block and for a refused block)
    int err;         // the lane's conversion or SwiGLU refusal (AH_ERR_*; 0: none)
    bool bad_block;  // quant_act refused the block (act_scale's None)
};
AH_DEV HiddenQ swiglu_quant32(uint32_t gate_bits, uint32_t up_bits, bool live) {
    HiddenQ o;
    o.err = 0;
    int64_t h = 0;
    if (live) {
        uint64_t mg, mu;
        bool ng, nu;
        int e = ah_to_q32_mag(gate_bits, mg, ng);
        if (!e) e = ah_to_q32_mag(up_bits, mu, nu);
        if (!e) e = swiglu_fx(ng ? (int64_t)(0ull - mg) : (int64_t)mg, nu ? (int64_t)(0ull - mu) : (int64_t)mu, h);
        if (e) {
            o.err = e;
            h = 0;
        }
    }
    const bool neg = h < 0;
    const uint64_t mag = neg ? 0ull - (uint64_t)h : (uint64_t)h;
    const int e = max32(mag ? ah_act_scale_exp(mag) : -1);
    bool bad = e == 63;  // act_scale's None
    const int c = e >= 0 && e < 63 ? ah_act_code(mag, neg, e, bad) : 0;
    const uint64_t group = 0xFFFFFFFFull << (threadIdx.x & 32);
    o.bad_block = (__builtin_amdgcn_ballot_w64(bad) & group) != 0ull;
    o.code = o.bad_block ? 0 : c;
    o.scale = o.bad_block || e < 0 ? 0ull : (1ull << e);
    return o;
}

}  // namespace
