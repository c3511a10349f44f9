// ah_units.h -- the GEMV's activation layout in LDS, the activation quantizer's quad helpers and
// the per-family dot units (Q8_0, Q5_0, Q2_K, Q3_K, Q4_K, Q6_K), shared by the streaming GEMV
// (ah_gemv.hip) and the GEMM's exact path for tokens the f16 operand cannot carry (ah_gemm.hip).
// A unit reads its weights through a generic pointer (an LDS tile in the GEMV, the GGUF row in
// global memory on the GEMM's exact path) and its activation from an ActLds.
#pragma once

#include "ah_internal.h"

namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// CP: cache policy of the load.  0 for inputs written before the launch; kCoherent (sc1, device
// scope) for inputs another workgroup of the same persistent launch wrote (gemv_seq_kernel).
constexpr int kCoherent = 16;
template <int CP = 0>
AH_DEV u32x2 ah_ld64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, CP));
}
template <int CP = 0>
AH_DEV u32x4 ah_ld128p(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, CP));
}

struct ActLds {
    int8_t *codes;   // [kpad]
    float *fsc;      // [kpad/32]   S_b * 2^-32
    float *fx32;     // [kpad/32]   fsc * X: the 32-block's code sum X times its scale (exact for a
                     //             power-of-two scale)
    int32_t *xs16;   // [kpad/16]   sum of codes per 16-group
    float *red;      // [1024]      unit partials of one tile (the tile copy follows)
};

// Activation codes sit in LDS with 16 bytes of padding after every 256: lanes working on
// consecutive super-blocks read codes 256 bytes apart, which would all map to one LDS bank.
AH_DEV uint32_t pad_k(uint32_t k) { return k + ((k >> 8) << 4); }
AH_DEV uint32_t codes_bytes(uint32_t kpad) { return kpad + kpad / 16; }

AH_DEV ActLds carve(uint8_t *smem, uint32_t kpad) {
    ActLds a;
    a.codes = reinterpret_cast<int8_t *>(smem);
    a.fsc = reinterpret_cast<float *>(smem + codes_bytes(kpad));
    a.fx32 = a.fsc + kpad / 32;
    a.xs16 = reinterpret_cast<int32_t *>(a.fx32 + kpad / 32);
    a.red = reinterpret_cast<float *>(a.xs16 + kpad / 16);
    return a;
}

// ---- activation quantizer: four lanes per 32-block ----------------------------------------------

// quad_perm DPP exchanges (VALU, no LDS): the value of lane ^1 / lane ^2 within each quad.
AH_DEV uint32_t quad_xor1(uint32_t v) { return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false); }
AH_DEV uint32_t quad_xor2(uint32_t v) { return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false); }

// One quad of lanes quantizes block b of an activation row (quant_act, chart/mod.rs:258-334);
// lane q = lane & 3 owns elements 8q .. 8q+7.  Every lane of the wave must call this together
// (the quad exchanges need all four lanes); `valid` is false for a block past the row.
// f32 input: to_q32 is monotone in |x|, so the block's largest f32 magnitude decides both the
// refusal and the scale.  Outputs: the lane's 8 codes packed in two dwords, its 16-element code
// sum (lanes 0/1: elements 0..15, lanes 2/3: 16..31), the 32-block sum, and the block exponent
// (-1: zero block).  Refusals are recorded with the index of the first failing element (input) or
// the block (quantizer), so the earliest refusal in element order wins, as in the reference.
struct QuadOut {
    uint32_t c0, c1;
    int s16, s32, e;
    float fsc;  // S_b * 2^-32 (0 for a zero or refused block)
};

// The raw inputs of one quad lane for one 32-block, loaded apart from the arithmetic so that a
// kernel can issue these loads ahead of its weight stream: 8 f32 bit patterns (w[0..7]), 8 Q32.32
// values (lo/hi in w[2i], w[2i+1]), or 8 int8 codes (w[0..1]) with the block scale (s0, s1).
// Words a source does not use may hold other bytes; its consumer never reads them.
struct QuadIn {
    uint32_t w[16];
    uint32_t s0, s1;  // codes: the block scale
    uint32_t take;
};
AH_DEV QuadIn quad_load(const void *x, const int64_t *scales, uint32_t src, uint32_t n_in, size_t row_off,
                        uint32_t b, bool valid) {
    QuadIn in;
    const uint32_t q = threadIdx.x & 3;
    const uint32_t k0 = b * 32 + 8 * q;
    in.take = (valid && n_in > k0) ? (n_in - k0 < 8 ? n_in - k0 : 8) : 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) in.w[i] = 0;
    if (src == AH_SRC_F32) {
        const uint32_t *xb = static_cast<const uint32_t *>(x) + row_off + k0;
        if (in.take == 8 && (reinterpret_cast<uintptr_t>(xb) & 15) == 0) {
            const u32x4 a = reinterpret_cast<const u32x4 *>(xb)[0], c = reinterpret_cast<const u32x4 *>(xb)[1];
            in.w[0] = a.x; in.w[1] = a.y; in.w[2] = a.z; in.w[3] = a.w;
            in.w[4] = c.x; in.w[5] = c.y; in.w[6] = c.z; in.w[7] = c.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) in.w[i] = (uint32_t)i < in.take ? xb[i] : 0u;
        }
    } else if (src == AH_SRC_Q32) {
        const uint64_t *xv = static_cast<const uint64_t *>(x) + row_off + k0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint64_t v = (uint32_t)i < in.take ? xv[i] : 0ull;
            in.w[2 * i] = (uint32_t)v;
            in.w[2 * i + 1] = (uint32_t)(v >> 32);
        }
    } else {
        const int8_t *c = static_cast<const int8_t *>(x) + row_off + k0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t v = (uint32_t)i < in.take ? (uint32_t)(uint8_t)c[i] : 0u;
            in.w[i >> 2] |= v << (8 * (i & 3));
        }
    }
    in.s0 = in.s1 = 0;
    if (src == AH_SRC_CODES && valid) {
        const uint64_t s = (uint64_t)scales[b];
        in.s0 = (uint32_t)s;
        in.s1 = (uint32_t)(s >> 32);
    }
    return in;
}

// The same inputs for one activation row of a GEMV read through buffer resources: elements past
// n_in lie past the resource's range and read as zero.  A GEMV's activation is f32 or codes (the
// Q32.32 form is the standalone quantizer's alone, which reads through quad_load).  Either source
// issues the same two 16-byte loads: the first 16 bytes of the lane's elements, then (resource
// and offset picked by `src` with scalar selects) f32 elements 4-7 or the codes' block scale with
// the next block's.  Their words land in w[4..7] and s0/s1 alike and each consumer reads only its
// own, so nothing here touches the loaded words: no branch, no copy and no wait (a branch between
// the sources' loads had made the compiler wait for the codes' scale before the weight loads went
// out), and no load out of range (those still take the vector memory path).  Codes are read a
// whole dword at a time (the base must be 4-byte aligned); quad_quant clears bytes past n_in.
struct ActRsrc {
    __amdgpu_buffer_rsrc_t x, s;
};
AH_DEV ActRsrc act_rsrc(const void *x, const int64_t *scales, uint32_t src, uint32_t n_in) {
    ActRsrc r;
    const uint32_t esz = src == AH_SRC_F32 ? 4u : src == AH_SRC_Q32 ? 8u : 1u;
    r.x = ah_rsrc(x, n_in * esz);
    r.s = ah_rsrc(scales, src == AH_SRC_CODES ? (n_in + 31) / 32 * 8 : 0u);
    return r;
}
constexpr uint32_t kActOob = 0xFFFFFFF0u;  // past any activation resource
template <int CP = 0>
AH_DEV QuadIn quad_load_row(const ActRsrc &r, uint32_t src, uint32_t n_in, uint32_t b) {
    QuadIn in;
    const uint32_t k0 = b * 32 + 8 * (threadIdx.x & 3);
    in.take = n_in > k0 ? (n_in - k0 < 8 ? n_in - k0 : 8) : 0;
    const bool f = src == AH_SRC_F32;
    const uint32_t base = f ? 4 * k0 : k0;
    const u32x4 l0 = ah_ld128p<CP>(r.x, base);
    const u32x4 l1 = ah_ld128p<CP>(f ? r.x : r.s, f ? base + 16 : 8 * b);
    in.w[0] = l0.x; in.w[1] = l0.y; in.w[2] = l0.z; in.w[3] = l0.w;
    in.w[4] = l1.x; in.w[5] = l1.y; in.w[6] = l1.z; in.w[7] = l1.w;
#pragma unroll
    for (int i = 8; i < 16; ++i) in.w[i] = 0u;
    in.s0 = l1.x;
    in.s1 = l1.y;
    return in;
}

// The common case of an f32 block, straight-line in f32 arithmetic: every block of the wave has
// its largest magnitude in [2^-9, 2^29) or is all zero (ballot-uniform; otherwise the whole wave
// takes the general form below).  Then no element is non-finite or past to_q32's range, and with
// the block's largest magnitude m * 2^(ee - 150) (m the 24-bit significand, ee in [118, 155]) its
// Q32.32 magnitude is m * 2^k, k = ee - 118, of bit length 24 + k: ah_act_scale_exp gives
// e = 17 + k + [m > 127 * 2^17], in [17, 55], so no code * 2^e leaves int64.
// Codes: v = |x| * 2^(32 - e) is exact (a power-of-two scaling, v <= 127, no underflow), and for
// |x| >= 2^-9 to_q32 is exact too, so the code is the one rounding floor(v + 1/2).  For v >= 1/2,
// floor(fl(v + 1/2)) is that value: v + 1/2 is exact while it stays in v's binade, and past it
// (in [2^j, 2^j + 1/2) for the next power 2^j) its rounding cannot reach the next integer.  Below
// 1/2 the code is 0, but fl(v + 1/2) rounds v = 1/2 - 2^-25 up to 1 (a tie, to even), so elements
// with |x| < 2^(e-33) (v < 1/2) are given 0 by a compare.  The sign rides on the addend:
// trunc(fl(x * 2^(32-e) + copysign(1/2, x))) = sign(x) * floor(fl(v + 1/2)), round-to-nearest
// being symmetric.  Below 2^-9, to_q32 rounds first: q = floor(fl(|x| * 2^32 + 1/2)), then the code
// rounds q * 2^-e the same way (q * 2^-e is a multiple of 2^-e >= 2^-24, so that sum is exact
// below 1; q itself is exact but at |x| * 2^32 = 1/2 - 2^-25, where it is 1 for 0, which no code
// at e >= 2 sees).  Both roundings give 0 when e >= 25 (q <= 2^23 < 2^(e-1)), so the second form
// runs only in waves with a block at e <= 24 (a largest magnitude below 1/2).
AH_DEV bool quad_quant_f32(const QuadIn &in, QuadOut &o) {
    uint32_t maxb = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) maxb = __builtin_elementwise_max(maxb, in.w[i] & 0x7fffffffu);
    maxb = __builtin_elementwise_max(maxb, quad_xor1(maxb));
    maxb = __builtin_elementwise_max(maxb, quad_xor2(maxb));
    const bool common = maxb == 0u || maxb - 0x3B000000u < 0x4E000000u - 0x3B000000u;
    if (__builtin_amdgcn_ballot_w64(!common) != 0ull) return false;
    const int e = maxb == 0u ? -1 : (int)(maxb >> 23) - 101 + ((maxb & 0x7fffffu) > 0x7E0000u ? 1 : 0);
    const float sc = __builtin_ldexpf(1.0f, 32 - e), half_unit = __builtin_ldexpf(1.0f, e - 33);
    int c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t w = in.w[i];
        const float x = __builtin_bit_cast(float, w);
        const int r = (int)__builtin_fmaf(x, sc, __builtin_bit_cast(float, (w & 0x80000000u) | 0x3F000000u));
        c[i] = __builtin_fabsf(x) >= half_unit ? r : 0;
    }
    if (__builtin_amdgcn_ballot_w64(e >= 0 && e <= 24) != 0ull) {
        const float se = __builtin_ldexpf(1.0f, -e);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t a = in.w[i] & 0x7fffffffu;
            const float qv = __builtin_floorf(__builtin_fmaf(__builtin_bit_cast(float, a), 0x1p32f, 0.5f));
            const int cm = (int)__builtin_fmaf(qv, se, 0.5f);
            if (a < 0x3B000000u) c[i] = (in.w[i] >> 31) ? -cm : cm;
        }
    }
    // low bytes of the codes, four to a dword (v_perm: bytes 0-3 of the second operand, 4-7 of the first)
    const uint32_t p01 = __builtin_amdgcn_perm((uint32_t)c[1], (uint32_t)c[0], 0x0c0c0400u);
    const uint32_t p23 = __builtin_amdgcn_perm((uint32_t)c[3], (uint32_t)c[2], 0x0c0c0400u);
    const uint32_t p45 = __builtin_amdgcn_perm((uint32_t)c[5], (uint32_t)c[4], 0x0c0c0400u);
    const uint32_t p67 = __builtin_amdgcn_perm((uint32_t)c[7], (uint32_t)c[6], 0x0c0c0400u);
    o.c0 = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
    o.c1 = __builtin_amdgcn_perm(p67, p45, 0x05040100u);
    const int s8 = ((c[0] + c[1]) + (c[2] + c[3])) + ((c[4] + c[5]) + (c[6] + c[7]));
    o.s16 = s8 + (int)quad_xor1((uint32_t)s8);
    o.s32 = o.s16 + (int)quad_xor2((uint32_t)o.s16);
    o.e = e;
    o.fsc = e < 0 ? 0.0f : __builtin_ldexpf(1.0f, e - 32);
    return true;
}

// fast: an f32 source tries quad_quant_f32 first; false keeps the general form only (a kernel
// whose register budget the fast form's temporaries would overflow).
AH_DEV QuadOut quad_quant(const QuadIn &in, uint32_t src, uint32_t b, unsigned long long *status,
                          unsigned long long key_base, bool fast = true) {
    const uint32_t q = threadIdx.x & 3;
    const uint32_t k0 = b * 32 + 8 * q;
    const uint32_t take = in.take;
    QuadOut o;
    if (fast && src == AH_SRC_F32 && quad_quant_f32(in, o)) return o;
    if (src == AH_SRC_CODES) {
        // precomputed codes (bytes past n_in cleared): only the code sums are derived here
        o.c0 = in.w[0] & (take >= 4 ? 0xffffffffu : (1u << (8 * take)) - 1u);
        o.c1 = in.w[1] & (take >= 8 ? 0xffffffffu : take <= 4 ? 0u : (1u << (8 * (take - 4))) - 1u);
        int s8 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) s8 += (int)(int8_t)((((i < 4) ? o.c0 : o.c1) >> (8 * (i & 3))) & 0xffu);
        o.s16 = s8 + (int)quad_xor1((uint32_t)s8);
        o.s32 = o.s16 + (int)quad_xor2((uint32_t)o.s16);
        o.e = 0;
        const int64_t S = (int64_t)(((uint64_t)in.s1 << 32) | in.s0);
        o.fsc = (float)S * 0x1p-32f;
        // QuantAct::dequantizes (chart/mod.rs:128-134): every S * code must be an i64, else the
        // call refuses with Dequant(FixedOverflow) before it projects.  A code is in [-128, 127],
        // so |S| <= 2^56 can never overflow (127 * 2^56 < 2^63, -128 * 2^56 = -2^63): the per-code
        // products are checked only in a wave with a larger scale (quantized activations have
        // S <= 2^57, past 2^56 only for magnitudes near 2^63).
        bool bad = false;
        const uint64_t mag = S < 0 ? 0ull - (uint64_t)S : (uint64_t)S;
        if (__builtin_amdgcn_ballot_w64(mag > (1ull << 56)) != 0ull) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                int64_t prod;
                bad |= __builtin_mul_overflow(S, (int64_t)(int8_t)((((i < 4) ? o.c0 : o.c1) >> (8 * (i & 3))) & 0xffu), &prod);
            }
        }
        const uint32_t badq = (uint32_t)bad | quad_xor1((uint32_t)bad);
        if ((badq | quad_xor2(badq)) != 0 && q == 0)
            ah_record(status, AH_QUANT_ORDER_BASE + (((key_base >> 5) + b) << 8) + 7u);
        return o;
    }
    uint32_t bits[8];
    int64_t v64[8];
    uint32_t maxb = 0;
    uint64_t maxm = 0;
    if (src == AH_SRC_F32) {
#pragma unroll
        for (int i = 0; i < 8; ++i) bits[i] = in.w[i];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t a = bits[i] & 0x7fffffffu;
            maxb = a > maxb ? a : maxb;
        }
        uint32_t t = quad_xor1(maxb);
        maxb = t > maxb ? t : maxb;
        t = quad_xor2(maxb);
        maxb = t > maxb ? t : maxb;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v64[i] = (int64_t)(((uint64_t)in.w[2 * i + 1] << 32) | in.w[2 * i]);
            const uint64_t m = v64[i] < 0 ? 0ull - (uint64_t)v64[i] : (uint64_t)v64[i];
            maxm = m > maxm ? m : maxm;
        }
        uint32_t lo = (uint32_t)maxm, hi = (uint32_t)(maxm >> 32);
        uint64_t t = ((uint64_t)quad_xor1(hi) << 32) | quad_xor1(lo);
        maxm = t > maxm ? t : maxm;
        lo = (uint32_t)maxm;
        hi = (uint32_t)(maxm >> 32);
        t = ((uint64_t)quad_xor2(hi) << 32) | quad_xor2(lo);
        maxm = t > maxm ? t : maxm;
    }
    o.c0 = o.c1 = 0;
    int s8 = 0;
    int e = -1;
    bool bad = false, refused = false;
    if (src == AH_SRC_F32) {
        bool mneg;
        if (ah_to_q32_mag(maxb, maxm, mneg) != 0) {
            // some element of the block is non-finite or out of range: record this lane's first
            refused = true;
            for (uint32_t i = 0; i < take; ++i) {
                uint64_t m;
                bool n;
                const int err = ah_to_q32_mag(bits[i], m, n);
                if (err) {
                    ah_record(status, ((key_base + k0 + i) << 8) | (unsigned)err);
                    break;
                }
            }
        }
    }
    if (!refused) {
        e = ah_act_scale_exp(maxm);
        bad = e == 63;
        if (e >= 0 && e < 63) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                int c;
                if (src == AH_SRC_F32) {
                    c = ah_act_code_f32(bits[i], e, bad);  // padded lanes are +0: code 0
                } else {
                    const bool n = v64[i] < 0;
                    const uint64_t m = n ? 0ull - (uint64_t)v64[i] : (uint64_t)v64[i];
                    c = ah_act_code(m, n, e, bad);
                }
                if (i < 4)
                    o.c0 |= (uint32_t)(c & 0xff) << (8 * i);
                else
                    o.c1 |= (uint32_t)(c & 0xff) << (8 * (i - 4));
                s8 += c;
            }
        }
    }
    // the dequantizes check is per block: any lane's failure refuses the whole block
    const uint32_t badq = (uint32_t)bad | quad_xor1((uint32_t)bad);
    const bool bad_block = (badq | quad_xor2(badq)) != 0;
    if (bad_block) {
        if (q == 0) ah_record(status, AH_QUANT_ORDER_BASE + (((key_base >> 5) + b) << 8) + 7u);
        o.c0 = o.c1 = 0;
        s8 = 0;
        e = -1;
    }
    if (refused) e = -1;
    o.s16 = s8 + (int)quad_xor1((uint32_t)s8);
    o.s32 = o.s16 + (int)quad_xor2((uint32_t)o.s16);
    o.e = e;
    o.fsc = e < 0 ? 0.0f : __builtin_ldexpf(1.0f, e - 32);
    return o;
}

AH_DEV QuadOut quant_quad(const void *x, uint32_t src, uint32_t n_in, size_t row_off, uint32_t b,
                          bool valid, unsigned long long *status, unsigned long long key_base) {
    return quad_quant(quad_load(x, nullptr, src, n_in, row_off, b, valid), src, b, status, key_base);
}

// Store one quad's block to the LDS activation.
// One per-block word per lane: lane 0 the scale, lane 2 the scaled block sum fsc * X, lanes 1 / 3
// their own 16-group sums (elements 0..15 / 16..31).  The words arrive as values (not through the QuadOut)
// so that the per-lane choice is a register select rather than a load from a chosen field.
AH_DEV void store_quad_words(const ActLds &A, uint32_t b, uint32_t c0, uint32_t c1, uint32_t fsc, uint32_t fx,
                             uint32_t s16) {
    const uint32_t q = threadIdx.x & 3;
    u32x2 *dst = reinterpret_cast<u32x2 *>(A.codes + pad_k(32 * b + 8 * q));
    *dst = (u32x2){c0, c1};
    uint32_t *const p = q == 0 ? reinterpret_cast<uint32_t *>(A.fsc) + b
                      : q == 2 ? reinterpret_cast<uint32_t *>(A.fx32) + b
                               : reinterpret_cast<uint32_t *>(A.xs16) + 2 * b + (q >> 1);
    *p = q == 0 ? fsc : q == 2 ? fx : s16;
}
AH_DEV void store_quad(const ActLds &A, uint32_t b, const QuadOut &o) {
    // |X| <= 32 * 128: (float)X is exact, and so is fsc * X when fsc is a power of two
    store_quad_words(A, b, o.c0, o.c1, __builtin_bit_cast(uint32_t, o.fsc),
                     __builtin_bit_cast(uint32_t, o.fsc * (float)o.s32), (uint32_t)o.s16);
}

// ---- per-family units, read from the LDS copy of the tile -------------------------------------

// Q8_0 block at byte `off` of the tile (format/quant.rs:238-250): f16 d at byte 0, 32 int8 codes
// at 2..33.  Blocks are 2-byte aligned: 9 dwords from the 4-aligned address below are realigned.
// DOTS: the debug entry point's exact group dots are stored (a runtime null check); without it the
// code has no store and no ragged-row case (blocks past n_in meet zero activations and add 0).
template <bool DOTS>
AH_DEV float unit_q8(const uint8_t *tl, uint32_t off, uint32_t b, const ActLds &A, int32_t *dots) {
    const uint32_t sh = off & 3u;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(tl + (off & ~3u));
    uint32_t w[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) w[i] = p[i];
    const uint32_t d16 = (sh ? (w[0] >> 16) : w[0]) & 0xffffu;
    const u32x4 *xv = reinterpret_cast<const u32x4 *>(A.codes + pad_k(32 * b));
    const u32x4 x0 = xv[0], x1 = xv[1];
    const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    int32_t D = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t c = sh ? w[i + 1] : ah_alignbyte(w[i + 1], w[i], 2);
        D = i == 0 ? ah_sdot4_first(c, xw[i]) : ah_sdot4(c, xw[i], D);
    }
    if (DOTS && dots) dots[b] = D;
    return ah_f16_bits_to_f32(d16) * A.fsc[b] * (float)D;
}

// Q5_0 block at byte `off` of the tile (format/quant.rs:261-297): f16 d at byte 0, the fifth bits
// qh (a little-endian u32) at 2..5, 16 bytes of nibbles at 6..21.  Output j < 16 is qs[j] & 15 with
// qh bit j as its fifth bit, output 16 + j is qs[j] >> 4 with qh bit 16 + j, each minus 16.  The
// five-bit values u (0..31) go to v_dot4 as bytes (four qh bits spread to bit 4 of four bytes by
// one multiply), and the -16 offset is folded through the block's code sum: D = sum u*xq - 16*X,
// applied as fsc * D = fsc * sum u*xq - 16 * fx32 (exact for a power-of-two fsc: both terms and
// their difference are representable).
template <bool DOTS>
AH_DEV float unit_q5(const uint8_t *tl, uint32_t off, uint32_t b, const ActLds &A, int32_t *dots) {
    const bool odd = (off & 3u) != 0;  // 2-byte aligned blocks: 6 dwords from the 4-aligned start
    const uint32_t *p = reinterpret_cast<const uint32_t *>(tl + (off & ~3u));
    uint32_t w[6];
#pragma unroll
    for (int i = 0; i < 6; ++i) w[i] = p[i];
    const uint32_t d16 = (odd ? (w[0] >> 16) : w[0]) & 0xffffu;
    const uint32_t qh = odd ? w[1] : ah_alignbyte(w[1], w[0], 2);
    const u32x4 *xv = reinterpret_cast<const u32x4 *>(A.codes + pad_k(32 * b));
    const u32x4 x0 = xv[0], x1 = xv[1];
    const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    int32_t D = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t qs = odd ? w[i + 2] : ah_alignbyte(w[i + 2], w[i + 1], 2);
        const uint32_t blo = ((((qh >> (4 * i)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
        const uint32_t bhi = ((((qh >> (16 + 4 * i)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
        D = i == 0 ? ah_sdot4_first((qs & 0x0F0F0F0Fu) | blo, xw[i]) : ah_sdot4((qs & 0x0F0F0F0Fu) | blo, xw[i], D);
        D = ah_sdot4(((qs >> 4) & 0x0F0F0F0Fu) | bhi, xw[4 + i], D);
    }
    if (DOTS && dots) {
        int32_t X = 0;  // the block's code sum, from the codes (the LDS holds it scaled)
#pragma unroll
        for (int i = 0; i < 8; ++i) X = ah_sdot4(0x01010101u, xw[i], X);
        dots[b] = D - 16 * X;
    }
    return ah_f16_bits_to_f32(d16) * __builtin_fmaf(-16.0f, A.fx32[b], A.fsc[b] * (float)D);
}

// Q4_K super-block s (format/quant.rs:481-510): d, dmin, 12 packed 6-bit (scale, min) pairs,
// 128 bytes of nibbles; sub-block j takes the low (j even) / high (j odd) nibbles of
// qs[32*(j/2) + l].  Term per sub-block: S_j * (d*sc_j*D_j - dmin*m_j*X_j).
//
// The eight (sc, m) pairs of get_scale_min_k4 (format/quant.rs:482-491) unpack as four words of
// four bytes each: sc 0-3 = b[0..3] & 63, m 0-3 = b[4..7] & 63, sc 4-7 = (b[8..11] & 15) |
// (b[0..3] >> 6) << 4, m 4-7 = (b[8..11] >> 4) | (b[4..7] >> 6) << 4.  sc_j * D_j is an exact
// integer (sc_j <= 63, |D_j| <= 32 * 15 * 128: below 2^22, one 24-bit multiply), so the unit sums
// S_j * (sc_j * D_j) and m_j * (S_j * X_j) (the activation's fx32) in f32, and d and dmin multiply
// once per unit.
struct Q4kScales {
    uint32_t sc[2], m[2];  // the bytes of sc 0-3, sc 4-7, m 0-3, m 4-7
};
AH_DEV Q4kScales q4k_scales(uint32_t s0, uint32_t s1, uint32_t s2) {
    Q4kScales q;
    q.sc[0] = s0 & 0x3F3F3F3Fu;
    q.m[0] = s1 & 0x3F3F3F3Fu;
    q.sc[1] = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    q.m[1] = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
    return q;
}
AH_DEV int32_t q4k_byte(uint32_t w, uint32_t k) { return (int32_t)((w >> (8 * k)) & 0xffu); }

// Pair P of a super-block (sub-blocks 2P, 2P + 1 from the low / high nibbles of qs[32P..32P+31]):
// adds its two terms to ad (S * sc * D) and am (m * S * X).
template <int P, bool DOTS>
AH_DEV void q4k_pair(const u32x4 *sb, const Q4kScales &q4, uint32_t g0, uint32_t nb32, const int8_t *cb,
                     int32_t *dots, float flo, float fhi, float xlo, float xhi, float &ad, float &am) {
    const u32x4 qa = sb[1 + 2 * P], qb = sb[2 + 2 * P];
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const u32x4 *xv = reinterpret_cast<const u32x4 *>(cb + 64 * P);  // pad_k(32 g0), g0 = 8s + 2P
    const u32x4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
    const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    int32_t Dlo = 0, Dhi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        Dlo = i == 0 ? ah_sdot4_first(q[i] & 0x0F0F0F0Fu, xl[i]) : ah_sdot4(q[i] & 0x0F0F0F0Fu, xl[i], Dlo);
        Dhi = i == 0 ? ah_sdot4_first((q[i] >> 4) & 0x0F0F0F0Fu, xh[i])
                     : ah_sdot4((q[i] >> 4) & 0x0F0F0F0Fu, xh[i], Dhi);
    }
    if (DOTS && dots) {
        dots[g0] = Dlo;
        if (g0 + 1 < nb32) dots[g0 + 1] = Dhi;  // a ragged row ends on an odd sub-block
    }
    const uint32_t scw = q4.sc[P >> 1], mw = q4.m[P >> 1], k = 2 * (P & 1);
    ad = __builtin_fmaf(flo, (float)__mul24(q4k_byte(scw, k), Dlo), ad);
    ad = __builtin_fmaf(fhi, (float)__mul24(q4k_byte(scw, k + 1), Dhi), ad);
    am = __builtin_fmaf((float)q4k_byte(mw, k), xlo, am);
    am = __builtin_fmaf((float)q4k_byte(mw, k + 1), xhi, am);
}
template <bool DOTS>
AH_DEV float unit_q4(const uint8_t *tl, uint32_t off, uint32_t s, uint32_t n_in, const ActLds &A,
                     int32_t *dots) {
    const u32x4 *sb = reinterpret_cast<const u32x4 *>(tl + off);  // 16-byte aligned
    const u32x4 h = sb[0];
    // the super-block's eight activation scales and scaled code sums, read ahead of the pairs
    float fs[8], fx[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        fs[i] = A.fsc[8 * s + i];
        fx[i] = A.fx32[8 * s + i];
    }
    const float fd = ah_f16_bits_to_f32(h.x & 0xffffu), fdm = ah_f16_bits_to_f32(h.x >> 16);
    const Q4kScales q4 = q4k_scales(h.y, h.z, h.w);
    const uint32_t nb32 = (n_in + 31) / 32, rem = n_in - 256 * s;
    // a ragged row's last super-block uses fewer pairs; without DOTS the rest meet zero activations
    const uint32_t npairs = !DOTS || rem >= 256 ? 4u : (rem + 63) / 64;
    const uint32_t g = 8 * s;
    float ad = 0.0f, am = 0.0f;
    const int8_t *const cb = A.codes + 272u * s;  // pad_k(32 * 8s): the super-block's codes
    q4k_pair<0, DOTS>(sb, q4, g, nb32, cb, dots, fs[0], fs[1], fx[0], fx[1], ad, am);
    if (npairs > 1) q4k_pair<1, DOTS>(sb, q4, g + 2, nb32, cb, dots, fs[2], fs[3], fx[2], fx[3], ad, am);
    if (npairs > 2) q4k_pair<2, DOTS>(sb, q4, g + 4, nb32, cb, dots, fs[4], fs[5], fx[4], fx[5], ad, am);
    if (npairs > 3) q4k_pair<3, DOTS>(sb, q4, g + 6, nb32, cb, dots, fs[6], fs[7], fx[6], fx[7], ad, am);
    return __builtin_fmaf(fd, ad, -(fdm * am));
}

// Q4_K in units of one pair of sub-blocks (64 elements; u = 4 s + P for super-block s and pair
// P), used where a projection is small enough that spreading a super-block over up to four lanes
// shortens its waves.  Pair P takes bytes 2(P & 1) and 2(P & 1) + 1 of the low (P < 2) or high
// (P >= 2) (sc, m) words above.
template <bool DOTS>
AH_DEV float unit_q4p(const uint8_t *tl, uint32_t off, uint32_t u, uint32_t n_in, const ActLds &A,
                      int32_t *dots) {
    const uint32_t P = u & 3u, g0 = 2 * u;  // pair P of super-block u / 4; its first 32-block
    const u32x4 *sb = reinterpret_cast<const u32x4 *>(tl + off);  // the super-block, 16-byte aligned
    const u32x4 h = sb[0];
    const u32x4 qa = sb[1 + 2 * P], qb = sb[2 + 2 * P];
    const float fd = ah_f16_bits_to_f32(h.x & 0xffffu), fdm = ah_f16_bits_to_f32(h.x >> 16);
    const bool hi47 = P >= 2;
    const uint32_t scw = hi47 ? ((h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u)) : (h.y & 0x3F3F3F3Fu);
    const uint32_t mw = hi47 ? (((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u)) : (h.z & 0x3F3F3F3Fu);
    const uint32_t k = 2 * (P & 1u);
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const u32x4 *xv = reinterpret_cast<const u32x4 *>(A.codes + pad_k(32 * g0));
    const u32x4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
    const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    int32_t Dlo = 0, Dhi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        Dlo = i == 0 ? ah_sdot4_first(q[i] & 0x0F0F0F0Fu, xl[i]) : ah_sdot4(q[i] & 0x0F0F0F0Fu, xl[i], Dlo);
        Dhi = i == 0 ? ah_sdot4_first((q[i] >> 4) & 0x0F0F0F0Fu, xh[i])
                     : ah_sdot4((q[i] >> 4) & 0x0F0F0F0Fu, xh[i], Dhi);
    }
    if (DOTS && dots) {
        const uint32_t nb32 = (n_in + 31) / 32;
        dots[g0] = Dlo;
        if (g0 + 1 < nb32) dots[g0 + 1] = Dhi;  // a ragged row ends on an odd 32-block
    }
    // (past a ragged row's end the codes are zero: the pair's second half adds nothing)
    const float ad = __builtin_fmaf(A.fsc[g0 + 1], (float)__mul24(q4k_byte(scw, k + 1), Dhi),
                                    A.fsc[g0] * (float)__mul24(q4k_byte(scw, k), Dlo));
    const float am = __builtin_fmaf((float)q4k_byte(mw, k + 1), A.fx32[g0 + 1], (float)q4k_byte(mw, k) * A.fx32[g0]);
    return __builtin_fmaf(fd, ad, -(fdm * am));
}

// Q6_K super-block s (format/quant.rs:556-599): ql[128] @0, qh[64] @128, int8 sc[16] @192,
// f16 d @208.  Element 128n + 32t + l = (nibble t/2 of ql[64n + 32(t&1) + l]
// | ((qh[32n + l] >> 2t) & 3) << 4) - 32.  The unit is one half n (128 elements: ql[64n..],
// qh[32n..], sc[8n..], d), so a row of K elements has ceil(K/128) units and a lane's work per
// unit is half a super-block.  Super-blocks are 2-byte aligned: the half's dwords are read from the
// 4-aligned address below and realigned.  The 6-bit value is built per word by one bit-field
// select (see below), and the block terms are exact integers folded in f32.
template <bool DOTS>
AH_DEV float unit_q6(const uint8_t *tl, uint32_t off, uint32_t s, uint32_t n, uint32_t n_in,
                     const ActLds &A, int32_t *dots16) {
    const uint32_t sh = off & 3u;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(tl + (off & ~3u));
    // the half's three regions as their own bases, so every read below has a constant offset
    const uint32_t *pl = p + 16 * n, *ph = p + 32 + 8 * n, *ps = p + 48 + 2 * n;
    const uint32_t nb32 = (n_in + 31) / 32, nb16 = (n_in + 15) / 16;
    auto V = [&](const uint32_t *b, int i) -> uint32_t { return ah_alignbyte(b[i + 1], b[i], sh); };
    const float fd = ah_f16_bits_to_f32(V(p, 52) & 0xffffu);
    float acc = 0.0f;
    const uint32_t scw[2] = {V(ps, 0), V(ps, 1)};
    // The qh pairs of a byte are bits (2t, 2t+1) for block t.  One mask per qh word keeps the
    // pairs of blocks 0 and 2 in place (bits 0-1, 4-5), one shift and mask brings those of blocks
    // 1 and 3 there; the 6-bit value is then (ql nibble) | (the pair moved to bits 4-5), one
    // bit-field insert after at most one shift per operand.  Blocks go in the order 0, 2, 1, 3,
    // so that only one of the two masked sets is live at a time.
    // the half's activation blocks g = 8s + 4n + t: pad_k(32 g) = 272 s + 128 n + 32 t (4n + t < 8),
    // so one base per unit and constant offsets per block
    const int8_t *const cb = A.codes + 272u * s + 128u * n;
    const int32_t *const x16 = A.xs16 + 16u * s + 8u * n;
    const float *const fb = A.fsc + 8u * s + 4u * n;
    uint32_t qm[8];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        const int t = tt == 1 ? 2 : tt == 2 ? 1 : tt;
        const uint32_t g = 8 * s + 4 * n + t;
        if (tt == 0 || tt == 2) {
#pragma unroll
            for (int i = 0; i < 8; ++i) qm[i] = ((t & 1) ? V(ph, i) >> 2 : V(ph, i)) & 0x33333333u;
        }
        if (DOTS && g >= nb32) continue;
        const u32x4 *xv = reinterpret_cast<const u32x4 *>(cb + 32 * t);
        const u32x4 x0 = xv[0], x1 = xv[1];
        const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        int32_t Dlo = 0, Dhi = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t qlw = V(pl, 8 * (t & 1) + i);
            const uint32_t lo = t < 2 ? qlw : qlw >> 4;    // the nibble at bits 0-3
            const uint32_t hi = t < 2 ? qm[i] << 4 : qm[i];  // the pair at bits 4-5 (6-7 clear)
            // (lo & 0x0F0F0F0F) | (hi & ~0x0F0F0F0F) as one v_bitop3 (table 0xE4: C ? A : B); the
            // builtin keeps the compiler from re-deriving the masks per block
            const uint32_t uu = __builtin_amdgcn_bitop3_b32(lo, hi, 0x0F0F0F0Fu, 0xE4);
            if (i < 4)
                Dlo = i == 0 ? ah_sdot4_first(uu, xw[i]) : ah_sdot4(uu, xw[i], Dlo);
            else
                Dhi = i == 4 ? ah_sdot4_first(uu, xw[i]) : ah_sdot4(uu, xw[i], Dhi);
        }
        Dlo -= 32 * x16[2 * t];
        Dhi -= 32 * x16[2 * t + 1];
        if (DOTS && dots16) {
            dots16[2 * g] = Dlo;
            if (2 * g + 1 < nb16) dots16[2 * g + 1] = Dhi;  // ragged row ends on a 16-group
        }
        const uint32_t sw = scw[t >> 1] >> (16 * (t & 1));
        // the block's two scale-weighted group dots as one integer (|sc * D| < 2^23, 24-bit
        // multiplies); d multiplies once per unit
        const int32_t I = __mul24((int)(int8_t)(sw & 0xffu), Dlo) + __mul24((int)(int8_t)((sw >> 8) & 0xffu), Dhi);
        acc = __builtin_fmaf(fb[t], (float)I, acc);
    }
    return fd * acc;
}

// Q2_K and Q3_K (format/quant.rs:308-476) in units of one half n of super-block s (128 elements,
// like Q6_K).  Element 128n + 32r + 16p + l takes bit pair r of qs[32n + 16p + l]; group j = 2r + p
// of the half is those 16 elements, consecutive in the activation.
//   Q2_K (84 bytes: scales[16] @0, qs @16, f16 d @80, f16 dmin @82; 4-byte aligned): group g's
//   byte scales[g] holds sc (low nibble) and m (high); term S * (d*sc*D - dmin*m*X) with D the
//   group's sum q*xq (q in 0..3) and X its code sum.
//   Q3_K (110 bytes: hmask[32] @0, qs @32, scales[12] @96, f16 d @108; 2-byte aligned, realigned
//   as Q6_K): the third bit of element (r, p, l) of half n is bit 4n + r of hmask[16p + l], and the
//   code is (q | hbit << 2) - 4; the 16 6-bit scales come from the 12 bytes by the kmask shuffle
//   (four little-endian words a0, a1, t: half n's groups 0-3 are ((a0 >> 4n) & 0x0F0F0F0F) |
//   ((t >> 4n) & 0x03030303) << 4, groups 4-7 the same from a1 and t >> (4n + 2)); term
//   S * d * (sc - 32) * D with D = sum (q | hbit << 2) * xq - 4 X.
// D is formed by four dot4 instructions per group on the masked bit pairs.
template <int TYPE, bool DOTS>
AH_DEV float unit_k23(const uint8_t *tl, uint32_t off, uint32_t s, uint32_t n, uint32_t n_in, const ActLds &A,
                      int32_t *dots16) {
    constexpr bool Q3 = TYPE == AH_GGML_Q3_K;
    const uint32_t sh = off & 3u;
    const uint32_t *p = reinterpret_cast<const uint32_t *>(tl + (off & ~3u));
    auto V = [&](int i) -> uint32_t { return Q3 ? ah_alignbyte(p[i + 1], p[i], sh) : p[i]; };
    float fd, fdm = 0.0f;
    uint32_t sw[2];
    if constexpr (Q3) {
        fd = ah_f16_bits_to_f32(V(27) & 0xffffu);
        const uint32_t a0 = V(24), a1 = V(25), t = V(26);
        sw[0] = ((a0 >> (4 * n)) & 0x0F0F0F0Fu) | (((t >> (4 * n)) & 0x03030303u) << 4);
        sw[1] = ((a1 >> (4 * n)) & 0x0F0F0F0Fu) | (((t >> (4 * n + 2)) & 0x03030303u) << 4);
    } else {
        const uint32_t dd = V(20);
        fd = ah_f16_bits_to_f32(dd & 0xffffu);
        fdm = ah_f16_bits_to_f32(dd >> 16);
        sw[0] = V(2 * n);
        sw[1] = V(2 * n + 1);
    }
    constexpr int kQs = Q3 ? 8 : 4;  // dword of qs[0]
    uint32_t q[8], hn[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        q[i] = V(kQs + 8 * (int)n + i);
        hn[i] = Q3 ? V(i) >> (4 * n) : 0u;  // this half's four hmask bits of each byte, at bits 0-3
    }
    const uint32_t nb16 = (n_in + 15) / 16;
    // The two 16-groups of a 32-block share its activation scale: their scale-weighted dots (and
    // Q2_K's min terms) are summed as integers, exactly (|sc * D| < 2^18 with 24-bit multiplies),
    // and each 32-block adds one f32 term per sum; d and dmin multiply once per unit.
    float aI = 0.0f, aM = 0.0f;
    int32_t Ip = 0, Mp = 0;
    // the half's 16-groups g = 16s + 8n + j: pad_k(16 g) = 272 s + 128 n + 16 j (8n + j < 16)
    const int8_t *const cb = A.codes + 272u * s + 128u * n;
    const int32_t *const x16 = A.xs16 + 16u * s + 8u * n;
    const float *const fb = A.fsc + 8u * s + 4u * n;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int r = j >> 1, pl = j & 1;
        const uint32_t g = 16 * s + 8 * n + (uint32_t)j;  // 16-group of the row
        if (DOTS && g >= nb16) break;
        const u32x4 xv = *reinterpret_cast<const u32x4 *>(cb + 16 * j);
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
        // Bit pairs r = 1, 2 are masked in place: each byte then holds its value times 4^r (at most
        // 7 * 16 = 112, still a positive int8), so the dot is 4^r D exactly and one shift recovers
        // D; pair 3 is shifted down first (in place it would read as negative bytes).  Q3_K's
        // hmask bit goes to the bit above the pair (hn: the half's bits moved to bits 0-3).
        int32_t D = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t qw = q[4 * pl + i];
            uint32_t v = r == 3 ? (qw >> 6) & 0x03030303u : qw & (0x03030303u << (2 * r));
            if constexpr (Q3) {
                const uint32_t hb = hn[4 * pl + i] & (0x01010101u << r);
                v |= r == 3 ? hb >> 1 : hb << (r + 2);
            }
            D = i == 0 ? ah_sdot4_first(v, xw[i]) : ah_sdot4(v, xw[i], D);
        }
        if (r == 1 || r == 2) D >>= 2 * r;
        const int32_t X = x16[j];
        const uint32_t sb = (sw[j >> 2] >> (8 * (j & 3))) & 0xffu;
        if constexpr (Q3) {
            D -= 4 * X;
            if (DOTS && dots16) dots16[g] = D;
            Ip += __mul24((int)sb - 32, D);
        } else {
            if (DOTS && dots16) dots16[g] = D;
            Ip += __mul24((int)(sb & 15u), D);
            Mp += __mul24((int)(sb >> 4), X);
        }
        // the 32-block's end (or, in the debug form, the ragged row's last group)
        if ((j & 1) || (DOTS && g + 1 >= nb16)) {
            const float f = fb[j >> 1];
            aI = __builtin_fmaf(f, (float)Ip, aI);
            if constexpr (!Q3) aM = __builtin_fmaf(f, (float)Mp, aM);
            Ip = 0;
            Mp = 0;
        }
    }
    return Q3 ? fd * aI : fd * aI - fdm * aM;
}

// Q4_K parts use pair units where the host chose them for a small projection (units = ceil(K/64)
// then exceeds the super-block count ceil(K/256); for K <= 64 the two forms are one).
AH_DEV bool q4k_pair_units(const GemvPart &P) { return P.units > (P.n_in + 255) / 256; }

// Unit u of the row that starts at byte `row_off` of the tile.  PAIRS: the kernel may meet Q4_K
// pair units (the latency launches' kernels); table plans and the workgroup-tile kernel never do.
template <int TYPE, bool DOTS, bool PAIRS = false>
AH_DEV float comp_unit(const GemvPart &P, const uint8_t *tl, uint32_t row_off, uint32_t row, uint32_t u,
                       const ActLds &A) {
    if constexpr (TYPE == AH_GGML_Q8_0) {
        const uint32_t nb32 = (P.n_in + 31) / 32;
        return unit_q8<DOTS>(tl, row_off + 34u * u, u, A, DOTS && P.dots ? P.dots + (size_t)row * nb32 : nullptr);
    } else if constexpr (TYPE == AH_GGML_Q5_0) {
        const uint32_t nb32 = (P.n_in + 31) / 32;
        return unit_q5<DOTS>(tl, row_off + 22u * u, u, A, DOTS && P.dots ? P.dots + (size_t)row * nb32 : nullptr);
    } else if constexpr (TYPE == AH_GGML_Q4_K) {
        const uint32_t nb32 = (P.n_in + 31) / 32;
        int32_t *dots = DOTS && P.dots ? P.dots + (size_t)row * nb32 : nullptr;
        if (PAIRS && q4k_pair_units(P)) return unit_q4p<DOTS>(tl, row_off + 144u * (u >> 2), u, P.n_in, A, dots);
        return unit_q4<DOTS>(tl, row_off + 144u * u, u, P.n_in, A, dots);
    } else if constexpr (TYPE == AH_GGML_Q2_K || TYPE == AH_GGML_Q3_K) {
        const uint32_t nb16 = (P.n_in + 15) / 16;
        return unit_k23<TYPE, DOTS>(tl, row_off + (TYPE == AH_GGML_Q2_K ? 84u : 110u) * (u >> 1), u >> 1, u & 1u,
                                    P.n_in, A, DOTS && P.dots ? P.dots + (size_t)row * nb16 : nullptr);
    } else {
        const uint32_t nb16 = (P.n_in + 15) / 16;
        return unit_q6<DOTS>(tl, row_off + 210u * (u >> 1), u >> 1, u & 1u, P.n_in, A,
                             DOTS && P.dots ? P.dots + (size_t)row * nb16 : nullptr);
    }
}

}  // namespace
