// ah_gemv.hip -- decode GEMV (N = 1) over GGUF Q8_0 / Q4_K / Q6_K payloads, and the activation
// quantizer passes.
//
// Reference semantics: matvec_q8act (chart/mod.rs:1887) equals matvec_fixed on the quantized
// activation; every row is the per-group fold acc += S_b * (w_scale*dot - w_min*xsum)
// (RowAcc::emit, chart/mod.rs:501-514) with exact integer group dots.  Here each dot is exact
// (v_dot4c_i32_i8) and the fold runs in f32 with the activation scale S_b * 2^-32 (a power of
// two, exact in f32) and the f16 weight scales (exact in f32).
//
// Work decomposition (HBM-bound).  A part's rows are cut into tiles of whole rows; a tile's
// (row, unit) pairs -- unit = one Q8_0 block or one K-quant super-block -- are flattened and
// dealt to the 256 threads of a workgroup (thread t takes units t, t+256, ..., NU per thread),
// so consecutive lanes read consecutive units of the GGUF bytes and no lane idles on a ragged
// row.  The first tile's weights are loaded before the activation prologue, and every tile's
// loads are issued before the previous tile is computed (double buffering in registers), so HBM
// latency overlaps the quantizer and the arithmetic.  Unit partials meet in LDS and each row is
// summed in a fixed order (deterministic output).
//
// The activation is quantized once per workgroup into LDS by one lane per 32-block (no
// cross-lane traffic): codes, per-32 f32 scale, per-32 and per-16 code sums.
#include "ah_internal.h"
#include "ah_swiglu.h"

namespace {

constexpr uint32_t kThreads = 256;

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
    int32_t *xs32;   // [kpad/32]   sum of codes per 32-block
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
    a.xs32 = reinterpret_cast<int32_t *>(a.fsc + kpad / 32);
    a.xs16 = a.xs32 + kpad / 32;
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
// One per-block word per lane: lane 0 the scale, lane 2 the block sum, lanes 1 / 3 their own
// 16-group sums (elements 0..15 / 16..31).  The words arrive as values (not through the QuadOut)
// so that the per-lane choice is a register select rather than a load from a chosen field.
AH_DEV void store_quad_words(const ActLds &A, uint32_t b, uint32_t c0, uint32_t c1, uint32_t fsc, uint32_t s32,
                             uint32_t s16) {
    const uint32_t q = threadIdx.x & 3;
    u32x2 *dst = reinterpret_cast<u32x2 *>(A.codes + pad_k(32 * b + 8 * q));
    *dst = (u32x2){c0, c1};
    uint32_t *const p = q == 0 ? reinterpret_cast<uint32_t *>(A.fsc) + b
                      : q == 2 ? reinterpret_cast<uint32_t *>(A.xs32) + b
                               : reinterpret_cast<uint32_t *>(A.xs16) + 2 * b + (q >> 1);
    *p = q == 0 ? fsc : q == 2 ? s32 : s16;
}
AH_DEV void store_quad(const ActLds &A, uint32_t b, const QuadOut &o) {
    store_quad_words(A, b, o.c0, o.c1, __builtin_bit_cast(uint32_t, o.fsc), (uint32_t)o.s32, (uint32_t)o.s16);
}

// Fill the LDS activation of part P: blocks past n_in (up to kpad) are zero, so ragged rows need
// no special case -- padded lanes contribute nothing to any dot or code sum.
AH_DEV void load_activation(const GemvPart &P, uint32_t kpad, const ActLds &A,
                            unsigned long long *status) {
    const uint32_t nbp = kpad / 32;
    const ActRsrc xr = act_rsrc(P.x, P.scales, P.src, P.n_in);
    for (uint32_t base = 0; base < nbp; base += kThreads / 4) {
        const uint32_t b = base + threadIdx.x / 4;
        const QuadOut o = quad_quant(quad_load_row(xr, P.src, P.n_in, b), P.src, b, status,
                                     (unsigned long long)P.key_tok * P.n_in);
        if (b < nbp) store_quad(A, b, o);
    }
}

// The workgroup's part: the launch argument, or its entry of a plan's part table.  The compiler
// reads either through one generic pointer into vector registers; every word is moved to a scalar
// register (the descriptor is the same for the whole workgroup), so buffer resources built from it
// are uniform and need no per-lane loop.
AH_DEV GemvPart load_part(const GemvPart &single, const GemvPart *__restrict__ parts,
                          const uint32_t *__restrict__ wg_part) {
    GemvPart P = parts ? parts[wg_part[blockIdx.x]] : single;
    static_assert(sizeof(GemvPart) % 4 == 0, "descriptor is whole dwords");
    uint32_t w[sizeof(GemvPart) / 4];
    __builtin_memcpy(w, &P, sizeof(P));
#pragma unroll
    for (uint32_t i = 0; i < sizeof(GemvPart) / 4; ++i) w[i] = __builtin_amdgcn_readfirstlane(w[i]);
    __builtin_memcpy(&P, w, sizeof(P));
    return P;
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
        D = ah_sdot4(c, xw[i], D);
    }
    if (DOTS && dots) dots[b] = D;
    return ah_f16_bits_to_f32(d16) * A.fsc[b] * (float)D;
}

// Q5_0 block at byte `off` of the tile (format/quant.rs:261-297): f16 d at byte 0, the fifth bits
// qh (a little-endian u32) at 2..5, 16 bytes of nibbles at 6..21.  Output j < 16 is qs[j] & 15 with
// qh bit j as its fifth bit, output 16 + j is qs[j] >> 4 with qh bit 16 + j, each minus 16.  The
// five-bit values u (0..31) go to v_dot4 as bytes (four qh bits spread to bit 4 of four bytes by
// one multiply), and the -16 offset is folded through the block's code sum: D = sum u*xq - 16*X.
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
        D = ah_sdot4((qs & 0x0F0F0F0Fu) | blo, xw[i], D);
        D = ah_sdot4(((qs >> 4) & 0x0F0F0F0Fu) | bhi, xw[4 + i], D);
    }
    D -= 16 * A.xs32[b];
    if (DOTS && dots) dots[b] = D;
    return ah_f16_bits_to_f32(d16) * A.fsc[b] * (float)D;
}

// Q4_K super-block s (format/quant.rs:481-510): d, dmin, 12 packed 6-bit (scale, min) pairs,
// 128 bytes of nibbles; sub-block j takes the low (j even) / high (j odd) nibbles of
// qs[32*(j/2) + l].  Term per sub-block: S_j * (d*sc_j*D_j - dmin*m_j*X_j).
//
// The eight (sc, m) pairs of get_scale_min_k4 (format/quant.rs:482-491) unpack as four words of
// four bytes each: sc 0-3 = b[0..3] & 63, m 0-3 = b[4..7] & 63, sc 4-7 = (b[8..11] & 15) |
// (b[0..3] >> 6) << 4, m 4-7 = (b[8..11] >> 4) | (b[4..7] >> 6) << 4.  d*sc_j and dmin*m_j are
// formed once per super-block; the per-sub-block arithmetic is f32 (no integer multiplies).
struct Q4kScales {
    float dsc[8], dm[8];
};
AH_DEV Q4kScales q4k_scales(uint32_t s0, uint32_t s1, uint32_t s2, float fd, float fdm) {
    const uint32_t sc03 = s0 & 0x3F3F3F3Fu, m03 = s1 & 0x3F3F3F3Fu;
    const uint32_t sc47 = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t m47 = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
    Q4kScales q;
    const uint32_t w[4] = {sc03, sc47, m03, m47};
    float b[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int k = 0; k < 4; ++k) b[4 * i + k] = (float)((w[i] >> (8 * k)) & 0xffu);  // v_cvt_f32_ubyteN
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        q.dsc[j] = fd * b[j];
        q.dm[j] = fdm * b[8 + j];
    }
    return q;
}

template <int P, bool DOTS>
AH_DEV float q4k_pair(const u32x4 *sb, const Q4kScales &q4, uint32_t g0, uint32_t nb32, const ActLds &A,
                      int32_t *dots, float flo, float fhi, float xlo, float xhi) {
    const u32x4 qa = sb[1 + 2 * P], qb = sb[2 + 2 * P];
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const u32x4 *xv = reinterpret_cast<const u32x4 *>(A.codes + pad_k(32 * g0));
    const u32x4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
    const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    int32_t Dlo = 0, Dhi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        Dlo = ah_sdot4(q[i] & 0x0F0F0F0Fu, xl[i], Dlo);
        Dhi = ah_sdot4((q[i] >> 4) & 0x0F0F0F0Fu, xh[i], Dhi);
    }
    if (DOTS && dots) {
        dots[g0] = Dlo;
        if (g0 + 1 < nb32) dots[g0 + 1] = Dhi;  // a ragged row ends on an odd sub-block
    }
    const float tlo = q4.dsc[2 * P] * (float)Dlo - q4.dm[2 * P] * xlo;
    const float thi = q4.dsc[2 * P + 1] * (float)Dhi - q4.dm[2 * P + 1] * xhi;
    return flo * tlo + fhi * thi;
}
template <bool DOTS>
AH_DEV float unit_q4(const uint8_t *tl, uint32_t off, uint32_t s, uint32_t n_in, const ActLds &A,
                     int32_t *dots) {
    const u32x4 *sb = reinterpret_cast<const u32x4 *>(tl + off);  // 16-byte aligned
    const u32x4 h = sb[0];
    // the super-block's eight activation scales and code sums, read ahead of the pairs
    float fs[8], xs[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        fs[i] = A.fsc[8 * s + i];
        xs[i] = (float)A.xs32[8 * s + i];  // |X| <= 32 * 128: exact
    }
    const float fd = ah_f16_bits_to_f32(h.x & 0xffffu), fdm = ah_f16_bits_to_f32(h.x >> 16);
    const Q4kScales q4 = q4k_scales(h.y, h.z, h.w, fd, fdm);
    const uint32_t nb32 = (n_in + 31) / 32, rem = n_in - 256 * s;
    // a ragged row's last super-block uses fewer pairs; without DOTS the rest meet zero activations
    const uint32_t npairs = !DOTS || rem >= 256 ? 4u : (rem + 63) / 64;
    const uint32_t g = 8 * s;
    float acc = q4k_pair<0, DOTS>(sb, q4, g, nb32, A, dots, fs[0], fs[1], xs[0], xs[1]);
    if (npairs > 1) acc += q4k_pair<1, DOTS>(sb, q4, g + 2, nb32, A, dots, fs[2], fs[3], xs[2], xs[3]);
    if (npairs > 2) acc += q4k_pair<2, DOTS>(sb, q4, g + 4, nb32, A, dots, fs[4], fs[5], xs[4], xs[5]);
    if (npairs > 3) acc += q4k_pair<3, DOTS>(sb, q4, g + 6, nb32, A, dots, fs[6], fs[7], xs[6], xs[7]);
    return acc;
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
    const uint32_t bsh = 16 * (P & 1u);
    const float sc0 = (float)((scw >> bsh) & 0xffu), sc1 = (float)((scw >> (bsh + 8)) & 0xffu);
    const float m0 = (float)((mw >> bsh) & 0xffu), m1 = (float)((mw >> (bsh + 8)) & 0xffu);
    const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const u32x4 *xv = reinterpret_cast<const u32x4 *>(A.codes + pad_k(32 * g0));
    const u32x4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
    const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    int32_t Dlo = 0, Dhi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        Dlo = ah_sdot4(q[i] & 0x0F0F0F0Fu, xl[i], Dlo);
        Dhi = ah_sdot4((q[i] >> 4) & 0x0F0F0F0Fu, xh[i], Dhi);
    }
    if (DOTS && dots) {
        const uint32_t nb32 = (n_in + 31) / 32;
        dots[g0] = Dlo;
        if (g0 + 1 < nb32) dots[g0 + 1] = Dhi;  // a ragged row ends on an odd 32-block
    }
    // (past a ragged row's end the codes are zero: the pair's second half adds nothing)
    const float tlo = (fd * sc0) * (float)Dlo - (fdm * m0) * (float)A.xs32[g0];
    const float thi = (fd * sc1) * (float)Dhi - (fdm * m1) * (float)A.xs32[g0 + 1];
    return A.fsc[g0] * tlo + A.fsc[g0 + 1] * thi;
}

// Q6_K super-block s (format/quant.rs:556-599): ql[128] @0, qh[64] @128, int8 sc[16] @192,
// f16 d @208.  Element 128n + 32t + l = (nibble t/2 of ql[64n + 32(t&1) + l]
// | ((qh[32n + l] >> 2t) & 3) << 4) - 32.  The unit is one half n (128 elements: ql[64n..],
// qh[32n..], sc[8n..], d), so a row of K elements has ceil(K/128) units and a lane's work per
// unit is half a super-block.  Super-blocks are 2-byte aligned: the half's dwords are read from the
// 4-aligned address below and realigned.  The 6-bit value is built with one and-or per word (the
// high bits are moved into place by one shift and mask), and the group terms are f32 (no integer
// multiplies).
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
    uint32_t qh[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) qh[i] = V(ph, i);
    const uint32_t scw[2] = {V(ps, 0), V(ps, 1)};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t g = 8 * s + 4 * n + t;
        if (DOTS && g >= nb32) break;
        const u32x4 *xv = reinterpret_cast<const u32x4 *>(A.codes + pad_k(32 * g));
        const u32x4 x0 = xv[0], x1 = xv[1];
        const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        int32_t Dlo = 0, Dhi = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t qlw = V(pl, 8 * (t & 1) + i);
            // bits 4-5 of each byte: qh bits 2t, 2t+1
            const uint32_t hi = (2 * t <= 4 ? (qh[i] << (4 - 2 * t)) : (qh[i] >> (2 * t - 4))) & 0x30303030u;
            const uint32_t uu = ((t < 2 ? qlw : (qlw >> 4)) & 0x0F0F0F0Fu) | hi;
            if (i < 4)
                Dlo = ah_sdot4(uu, xw[i], Dlo);
            else
                Dhi = ah_sdot4(uu, xw[i], Dhi);
        }
        Dlo -= 32 * A.xs16[2 * g];
        Dhi -= 32 * A.xs16[2 * g + 1];
        if (DOTS && dots16) {
            dots16[2 * g] = Dlo;
            if (2 * g + 1 < nb16) dots16[2 * g + 1] = Dhi;  // ragged row ends on a 16-group
        }
        const uint32_t sw = scw[t >> 1] >> (16 * (t & 1));
        // the block's two scale-weighted group dots as one integer (|sc * D| < 2^23, 24-bit
        // multiplies); d multiplies once per unit
        const int32_t I = __mul24((int)(int8_t)(sw & 0xffu), Dlo) + __mul24((int)(int8_t)((sw >> 8) & 0xffu), Dhi);
        acc = __builtin_fmaf(A.fsc[g], (float)I, acc);
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
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int r = j >> 1, pl = j & 1;
        const uint32_t g = 16 * s + 8 * n + (uint32_t)j;  // 16-group of the row
        if (DOTS && g >= nb16) break;
        const u32x4 xv = *reinterpret_cast<const u32x4 *>(A.codes + pad_k(16 * g));
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
            D = ah_sdot4(v, xw[i], D);
        }
        if (r == 1 || r == 2) D >>= 2 * r;
        const int32_t X = A.xs16[g];
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
            const float f = A.fsc[g >> 1];
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

constexpr uint32_t kRedSlots = 1024;  // unit partials of one tile
constexpr uint32_t kTileSlack = 128;  // bytes past a tile that realigned or compact-row unit reads may touch

// One workgroup streams whole-row tiles of a part.  A tile's bytes are loaded with 16-byte
// buffer loads in which consecutive lanes take consecutive chunks (each wave instruction reads
// 1 KB contiguous), held in registers until the previous tile is done, then copied to LDS; each
// lane then reads its (row, unit) pairs out of LDS.  The next tile's loads are issued as soon as
// the current tile reaches LDS, so they overlap its arithmetic and reduction.
template <int TYPE, int NC>
__global__ void __launch_bounds__(kThreads)
    gemv_kernel(GemvPart single, const GemvPart *__restrict__ parts,
                const uint32_t *__restrict__ wg_part, uint32_t kpad_max,
                unsigned long long *status) {
    extern __shared__ __align__(16) uint8_t smem[];
    const GemvPart P = load_part(single, parts, wg_part);
    const uint32_t wg_local = blockIdx.x - P.wg_begin;
    const uint32_t kpad = (P.n_in + 255) / 256 * 256;
    const ActLds A = carve(smem, kpad_max);
    uint8_t *tl = reinterpret_cast<uint8_t *>(A.red + kRedSlots);
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(P.w, (uint32_t)P.w_bytes);
    const uint32_t U = P.units, R = P.rows_per_tile, TU = R * U, RB = P.row_bytes;
    const uint32_t n_tiles = (P.n_out + R - 1) / R;

    u32x4 chunk[NC];
    auto load_tile = [&](uint32_t tile) {
        const uint32_t start = tile * R * RB;
        const uint32_t rows = P.n_out - tile * R < R ? P.n_out - tile * R : R;
        const uint32_t a0 = start & ~15u;
        const uint32_t nch = (rows * RB + (start - a0) + 15) / 16;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const uint32_t c = threadIdx.x + kThreads * i;
            chunk[i] = c < nch ? ah_ld128_nt(rs, a0 + 16 * c) : (u32x4){0u, 0u, 0u, 0u};
        }
    };

    uint32_t tile = wg_local;
    if (tile < n_tiles) load_tile(tile);
    load_activation(P, kpad, A, status);

    for (; tile < n_tiles; tile += P.wg_count) {
        ah_lds_barrier();  // the previous tile is consumed; the activation is in LDS
#pragma unroll
        for (int i = 0; i < NC; ++i) reinterpret_cast<u32x4 *>(tl)[threadIdx.x + kThreads * i] = chunk[i];
        const uint32_t next = tile + P.wg_count;
        if (next < n_tiles) load_tile(next);
        ah_lds_barrier();
        const uint32_t toff = (tile * R * RB) & 15u;
        for (uint32_t f = threadIdx.x; f < TU; f += kThreads) {
            const uint32_t r = f / U, u = f - r * U, row = tile * R + r;
            float v = 0.0f;
            if (row < P.n_out) v = comp_unit<TYPE, true>(P, tl, toff + r * RB, row, u, A);
            A.red[f] = v;
        }
        ah_lds_barrier();
        // row sums in fixed order: G lanes per row, G a power of two with R*G <= 256
        uint32_t G = 64;
        while (G > 1 && R * G > kThreads) G >>= 1;
        const uint32_t r = threadIdx.x / G, gl = threadIdx.x & (G - 1);
        float sum = 0.0f;
        if (r < R)
            for (uint32_t i = gl; i < U; i += G) sum += A.red[r * U + i];
        for (uint32_t o = 1; o < G; o <<= 1) sum += __shfl_xor(sum, (int)o, 64);
        const uint32_t row = tile * R + r;
        if (r < R && gl == 0 && row < P.n_out) {
            P.y[row] = sum;
            const uint32_t oc = ah_out_code(sum);
            if (oc) ah_record(status, ah_out_key(P.out_key0 + row, oc));
        }
    }
}

// Standalone quantizer: one quad of lanes per (token, 32-block) -- quant_act per token row,
// bit-exact.  The loop trip count is uniform so every quad exchange has all four lanes.
__global__ void __launch_bounds__(kThreads) quant_kernel(QuantArgs q) {
    const size_t total = (size_t)q.n_tok * q.nb32;
    const size_t stride = (size_t)gridDim.x * (kThreads / 4);
    for (size_t base = (size_t)blockIdx.x * (kThreads / 4); base < total; base += stride) {
        const size_t i = base + threadIdx.x / 4;
        const bool valid = i < total;
        const uint32_t tok = valid ? (uint32_t)(i / q.nb32) : 0, b = valid ? (uint32_t)(i % q.nb32) : 0;
        const QuadOut o = quant_quad(q.x, q.src, q.n_in, (size_t)tok * q.n_in, b, valid, q.status,
                                     (unsigned long long)tok * q.n_in);
        if (!valid) continue;
        const uint32_t lq = threadIdx.x & 3, k0 = 32 * b + 8 * lq;
        int8_t *dst = q.codes + (size_t)tok * q.n_in + k0;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k0 + k < q.n_in) dst[k] = (int8_t)(((k < 4 ? o.c0 : o.c1) >> (8 * (k & 3))) & 0xffu);
        if (lq == 0) q.scales[(size_t)tok * q.nb32 + b] = o.e < 0 ? 0 : (int64_t)(1ull << o.e);
    }
}

// Largest value over the wave (every lane gets it).
AH_DEV int wave_max(int v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_xor(v, o, 64);
        v = t > v ? t : v;
    }
    return v;
}
AH_DEV int wave_min(int v) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_xor(v, o, 64);
        v = t < v ? t : v;
    }
    return v;
}
// GEMM activation operand straight from the input, one workgroup per token.  Every 32-block is
// quantized once, bit-exactly (quant_act, chart/mod.rs:258-334; refusals recorded as quant_kernel
// does).  The token's largest block exponent E is the max of the block exponents (act_scale is
// monotone in absmax, kern/pow2.rs:11-39); with it the kernel writes
//   xh   = xq * 2^(e_b - E) in f16 (exact whenever e_b - E >= -24),
//   tok_scale = 2^(E - 32),
//   xmin (Q4_K) = per 32-block code sum X split exactly as [64*floor(X/64), X mod 64] * 2^(e_b - E),
//        laid out per super-block as [hi 0..7, lo 0..7].
// With codes input (AH_SRC_CODES) the block exponents come from the power-of-two scales.
// A quad of lanes owns a block per round and R rounds cover the padded row, so every input load
// of the token is issued before the first is used and the quantized blocks stay in registers: one
// memory round trip, one reduction of E, then the stores.  Rows past 64 blocks (K > 2048) take
// 1024-thread workgroups: 16 waves per token keep a CU's 32 wave slots full at prefill sizes,
// where 4 waves per token left the exact quantizer's VALU work and the load latency exposed.

// One quad lane's inputs for block b, issuing only the loads its source kind needs: two 16-byte
// loads of f32, or 8 code bytes plus the block scale (dword loads: the row must start on a 4-byte
// boundary, i.e. n_in % 4 == 0).  Past n_in the resource reads zeros.
template <uint32_t SRC>
AH_DEV QuadIn operand_load(const ActRsrc &r, uint32_t n_in, uint32_t b) {
    QuadIn in;
    const uint32_t k0 = b * 32 + 8 * (threadIdx.x & 3);
    in.take = n_in > k0 ? (n_in - k0 < 8 ? n_in - k0 : 8) : 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) in.w[i] = 0;
    in.s0 = in.s1 = 0;
    if constexpr (SRC == AH_SRC_F32) {
        const u32x4 l0 = ah_ld128(r.x, 4 * k0), l1 = ah_ld128(r.x, 4 * k0 + 16);
        in.w[0] = l0.x; in.w[1] = l0.y; in.w[2] = l0.z; in.w[3] = l0.w;
        in.w[4] = l1.x; in.w[5] = l1.y; in.w[6] = l1.z; in.w[7] = l1.w;
    } else {
        const u32x2 c = ah_ld64(r.x, k0), sc = ah_ld64(r.s, 8 * b);
        in.w[0] = c.x;
        in.w[1] = c.y;
        in.s0 = sc.x;
        in.s1 = sc.y;
    }
    return in;
}

template <uint32_t SRC, uint32_t R, uint32_t T>
__global__ void __launch_bounds__(T) gemm_operand_kernel(OperandArgs o) {
    static_assert(SRC == AH_SRC_F32 || SRC == AH_SRC_CODES, "the GEMM takes f32 or code inputs");
    constexpr uint32_t kOpBlocks = T / 4;  // blocks per round
    __shared__ uint32_t red[T / 64], redn[T / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = tid & 3;
    const uint32_t tok = blockIdx.x;
    const size_t row = (size_t)tok * o.n_in;
    const uint32_t esz = SRC == AH_SRC_F32 ? 4u : 1u;
    const int64_t *srow = SRC == AH_SRC_CODES ? o.scales + (size_t)tok * o.nb32 : nullptr;
    const ActRsrc r = act_rsrc(static_cast<const uint8_t *>(o.x) + row * esz, srow, SRC, o.n_in);
    const uint32_t nbp = o.kpad / 32;
    // codes rows start at tok * n_in bytes: bytewise loads unless that is a dword boundary
    const bool bytewise = SRC == AH_SRC_CODES && (o.n_in & 3u) != 0;
    // a wave whose first block of round u is past the padded row skips the round (and the later
    // ones): every lane's block would read zeros
    const uint32_t wb0 = __builtin_amdgcn_readfirstlane(wave) * 16u;
    QuadIn in[R];
#pragma unroll
    for (uint32_t u = 0; u < R; ++u) {
        if (u * kOpBlocks + wb0 >= nbp) break;
        const uint32_t b = u * kOpBlocks + tid / 4;
        in[u] = bytewise ? quad_load(o.x, srow, SRC, o.n_in, row, b, b < o.nb32) : operand_load<SRC>(r, o.n_in, b);
    }
    uint32_t c0[R], c1[R];
    int ex[R], sum[R], sum16[R];
    int emax = -1, emin = 64;  // largest block exponent, smallest of a nonzero block
    bool odd = false;          // a codes scale that is not a power of two
#pragma unroll
    for (uint32_t u = 0; u < R; ++u) {
        if (u * kOpBlocks + wb0 >= nbp) break;
        const uint32_t b = u * kOpBlocks + tid / 4;
        const QuadOut qo = quad_quant(in[u], SRC, b, o.status, (unsigned long long)row);
        int e = qo.e;
        if (SRC == AH_SRC_CODES) {
            const uint64_t S = ((uint64_t)in[u].s1 << 32) | in[u].s0;
            e = (int64_t)S > 0 ? 63 - __builtin_clzll(S) : -1;
            // a QuantAct built by hand may hold any i64 scale: one that is not 0 or a power of
            // two has no exact f16 operand, so the token takes the exact path
            if (S != 0 && ((int64_t)S < 0 || (S & (S - 1)) != 0)) { e = 0; odd = true; }
        }
        if (b >= nbp) e = -1;
        c0[u] = qo.c0;
        c1[u] = qo.c1;
        ex[u] = e;
        sum[u] = qo.s32;
        sum16[u] = qo.s16;
        emax = e > emax ? e : emax;
        emin = e >= 0 && e < emin ? e : emin;
    }
    emax = wave_max(emax);
    emin = wave_min(odd ? -1000 : emin);  // below any band: the token is flagged
    if (lane == 0) {
        red[wave] = (uint32_t)(emax + 1);
        redn[wave] = (uint32_t)emin;
    }
    __syncthreads();
    int E = -1, Emin = 64;
#pragma unroll
    for (uint32_t w = 0; w < T / 64; ++w) {
        E = (int)red[w] - 1 > E ? (int)red[w] - 1 : E;
        Emin = (int)redn[w] < Emin ? (int)redn[w] : Emin;
    }
    if (E > 62) E = 62;  // a block without a Q32.32 scale: the call is refused anyway
    // a nonzero block below the f16 band (when the f16 operand is written; the int8 design's
    // bf16 block factors carry any gap), or a scale that is not a power of two: the GEMM serves
    // this token exactly from its codes
    const bool flagged = (o.xh || o.xf) ? Emin < E - kF16Band : Emin < -500;
    if (tid == 0) {
        const float ts = E < 0 ? 0.0f : __builtin_ldexpf(1.0f, E - 32);
        o.tok_scale[tok] = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, ts) | (flagged ? 1u : 0u));
    }
    if (SRC == AH_SRC_F32 && flagged) {
        // keep the token's QuantAct for the exact path (uniform branch: one workgroup per token)
        int8_t *fc = o.fcodes + row;
        int64_t *fs = o.fscales + (size_t)tok * o.nb32;
#pragma unroll
        for (uint32_t u = 0; u < R; ++u) {
            if (u * kOpBlocks + wb0 >= nbp) break;
            const uint32_t b = u * kOpBlocks + tid / 4;
            if (b >= o.nb32) continue;
            const uint32_t k0 = 32 * b + 8 * q;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (k0 + i < o.n_in) fc[k0 + i] = (int8_t)(((i < 4 ? c0[u] : c1[u]) >> (8 * (i & 3))) & 0xffu);
            if (q == 0) fs[b] = ex[u] < 0 ? 0 : (int64_t)(1ull << ex[u]);
        }
    }
    if (o.xc) {
        // int8 design: the codes (zero past n_in) and the block factor 2^(e_b - E) as a bf16 pair
        int8_t *xc = o.xc + (size_t)tok * o.kpad;
        uint32_t *xsp = o.xsp + (size_t)tok * nbp;
#pragma unroll
        for (uint32_t u = 0; u < R; ++u) {
            if (u * kOpBlocks + wb0 >= nbp) break;
            const uint32_t b = u * kOpBlocks + tid / 4;
            if (b >= nbp) continue;
            const u32x2 cv = {c0[u], c1[u]};
            *reinterpret_cast<u32x2 *>(xc + 32 * b + 8 * q) = cv;
            if (q == 0) {
                const uint32_t bf = ex[u] < 0 ? 0u : (uint32_t)(ex[u] - E + 127) << 7;  // 2^(e-E) >= 2^-63
                xsp[b] = bf | (bf << 16);
            }
        }
    }
    if (!o.xh && !o.xf) return;
    _Float16 *xh = o.xh ? o.xh + (size_t)tok * o.kpad : nullptr;
    // fragment order: token tok's 16 bytes of K chunk k0 = 32 b + 8 q sit in block (tok / 32, k0 / 16)
    // at lane 32 ((k0 / 8) & 1) + tok % 32
    _Float16 *xf = o.xf ? o.xf + ((size_t)(tok / 32) * (o.kpad / 16)) * 512 + (tok % 32) * 8 : nullptr;
#pragma unroll
    for (uint32_t u = 0; u < R; ++u) {
        if (u * kOpBlocks + wb0 >= nbp) break;
        const uint32_t b = u * kOpBlocks + tid / 4;
        if (b >= nbp) continue;
        const int e = ex[u], sh = e - E;
        _Float16 hv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = (int)(int8_t)(((i < 4 ? c0[u] : c1[u]) >> (8 * (i & 3))) & 0xffu);
            hv[i] = e < 0 ? (_Float16)0.0f : (_Float16)__builtin_ldexpf((float)c, sh);
        }
        if (xh) *reinterpret_cast<u32x4 *>(xh + 32 * b + 8 * q) = __builtin_bit_cast(u32x4, hv);
        if (xf) {
            const uint32_t k0 = 32 * b + 8 * q;
            *reinterpret_cast<u32x4 *>(xf + (size_t)(k0 / 16) * 512 + 256 * ((k0 / 8) & 1)) = __builtin_bit_cast(u32x4, hv);
        }
        if (o.xmin16 && (q & 1u) == 0) {
            // lanes 0 and 2 hold the sums of the block's 16-groups 2 (b % 8) and 2 (b % 8) + 1
            _Float16 *m = o.xmin16 + ((size_t)tok * (o.kpad / 256) + b / 8) * 16;
            m[2 * (b % 8) + (q >> 1)] = e < 0 ? (_Float16)0.0f : (_Float16)__builtin_ldexpf((float)sum16[u], sh);
        }
        if (o.xmin && q == 0) {
            const int X = sum[u];
            const int hq = (X >= 0 ? X : X - 63) / 64;  // floor(X / 64)
            _Float16 *m = o.xmin + ((size_t)tok * (o.kpad / 256) + b / 8) * 16;
            m[b % 8] = e < 0 ? (_Float16)0.0f : (_Float16)__builtin_ldexpf((float)(64 * hq), sh);
            m[8 + b % 8] = e < 0 ? (_Float16)0.0f : (_Float16)__builtin_ldexpf((float)(X - 64 * hq), sh);
        }
    }
}

// Device-side f16 scale scan of a payload: records the earliest Inf/NaN d / dmin word as
// (block << 17) | (dmin << 16) | bits.
__global__ void scan_scales_kernel(const uint8_t *w, uint64_t n_blocks, uint32_t block_bytes,
                                   uint32_t off0, uint32_t off1, unsigned long long *bad) {
    for (uint64_t b = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; b < n_blocks;
         b += (uint64_t)gridDim.x * blockDim.x) {
        const uint8_t *p = w + b * block_bytes;
        const uint32_t h0 = p[off0] | (p[off0 + 1] << 8);
        const uint32_t h1 = off1 != off0 ? (uint32_t)(p[off1] | (p[off1 + 1] << 8)) : 0u;
        if (((h0 >> 10) & 0x1f) == 0x1f) atomicMin(bad, (b << 17) | h0);
        else if (((h1 >> 10) & 0x1f) == 0x1f) atomicMin(bad, (b << 17) | (1ull << 16) | h1);
    }
}

}  // namespace

// ---- launchers (called from ah_abi.cpp) ----

// ---- streaming GEMV ---------------------------------------------------------------------------
//
// Each wave owns a contiguous range of whole rows of its part (the part's rows split evenly over
// its waves) and streams them in tiles of whole rows, at most kStreamTile bytes each.  A tile is
// read with 16-byte buffer loads in which lane l takes chunks l, l+64, ... (each load instruction
// reads 1 KB contiguous; a chunk past the tile takes an out-of-range offset and reads nothing),
// held in registers while the wave computes the previous tile from its LDS slot, then written to
// the slot.  Eight waves share a workgroup and its quantized activation; the tile loop has no
// workgroup barrier.
//
// The activation loads go out before the first tile's, so waiting for them does not wait for the
// weights, and the quantizer runs while the first tile streams in.
//
// A row is owned by G = P.lanes consecutive lanes, lane g taking units g, g+G, ...; the G partial
// sums meet through DPP row operations (and, for G > 16, lane shuffles) in a fixed order.

template <int CTRL, int ROWS = 0xF>
AH_DEV float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF, false));
}
// Sum over aligned groups of G lanes (G a power of two <= 64), in the group's last lane
// (g = G - 1).  Up to 16 lanes the butterflies stay within a DPP row and every lane gets the sum;
// for 32 and 64 the rows' sums are folded upward by row broadcasts (VALU, no LDS permute): lane 15
// of rows 0 / 2 into rows 1 / 3, then lane 31 into rows 2 and 3 (rows outside the mask keep theirs).
AH_DEV float group_sum(float s, uint32_t G) {
    if (G >= 2) s += dpp<0xB1>(s);        // quad_perm [1,0,3,2]: lane ^ 1
    if (G >= 4) s += dpp<0x4E>(s);        // quad_perm [2,3,0,1]: lane ^ 2
    if (G >= 8) s += dpp<0x141>(s);       // row_half_mirror: the other quad of the half-row
    if (G >= 16) s += dpp<0x140>(s);      // row_mirror: the other half of the row
    if (G >= 32) s += dpp<0x142, 0xA>(s); // row_bcast:15 into rows 1 and 3
    if (G >= 64) s += dpp<0x143, 0xC>(s); // row_bcast:31 into rows 2 and 3
    return s;
}


constexpr uint32_t kSThreads = 512;                // threads of a streaming workgroup
constexpr uint32_t kSWaves = kSThreads / 64;
constexpr uint32_t kChunks = 8;                    // 16-byte loads per lane per tile
constexpr uint32_t kStreamTile = kChunks * 1024;   // bytes per tile
constexpr uint32_t kSlotBytes = kStreamTile + 128; // + what realigned or compact-row unit reads touch past a tile
constexpr uint32_t kOob = 0xFFFFFFF0u;             // past any payload (payloads stay below 4 GiB - 256)

// Part descriptor `i` of a plan's table, every word in a scalar register.
AH_DEV GemvPart part_at(const GemvPart *__restrict__ parts, uint32_t i) {
    GemvPart P = parts[i];
    uint32_t w[sizeof(GemvPart) / 4];
    __builtin_memcpy(w, &P, sizeof(P));
#pragma unroll
    for (uint32_t k = 0; k < sizeof(GemvPart) / 4; ++k) w[k] = __builtin_amdgcn_readfirstlane(w[k]);
    __builtin_memcpy(&P, w, sizeof(P));
    return P;
}

// PLAN: each wave's part and rows come from the workgroup's StreamWG entry (read with scalar
// loads, which do not queue behind the vector memory stream), and the workgroup first quantizes
// the activations of all its waves' parts.  Otherwise every wave serves the launch argument's
// part, its rows split evenly over the grid's waves.  Otherwise each workgroup serves one of the
// argument parts (whole workgroups per part), its rows split evenly over that part's waves.
// TYPE kMixedType: the parts may be of different GGUF types; each wave's units are
// computed by the loop of its part's type, a branch that is uniform over the wave and taken once
// per tile outside the unit loop.  The activation layout is the same for every type.
// DOTS: the debug form that also stores exact group dots (single launches only).
// LDS: [activation region: act_bytes][one tile slot per wave].
// Single-type kernels run 4 waves per SIMD (two workgroups per CU, <= 128 VGPRs).  The mixed-type
// kernel holds every type's unit loop and spilled at that budget (1.1 MB of scratch writes per
// configs[4] q/k/v launch); its plans are small (36 workgroups for q/k/v), so it is built for 2
// waves per SIMD (one workgroup per CU, <= 256 VGPRs), which costs those plans nothing.
template <int TYPE>
constexpr int stream_waves_per_simd() { return TYPE == kMixedType ? 2 : 4; }

// LDS of the fused FFN's gate/up launch past the tile slots: the gate and up row sums (f32) of
// the workgroup's hidden blocks.
constexpr uint32_t kFfnRows = 32 * kFfnMaxBlocks;
constexpr uint32_t kFfnLdsBytes = 2 * kFfnRows * 4;


// The fused FFN's epilogue over the workgroup's hidden blocks [b0, b1): one thread per element,
// 32 lanes per block.  Each converts its gate and up row sums to Q32.32 (to_q32) and forms
// h = round_shift_32(silu_fixed(gate) * up) (engine/ops/ffn.rs:80, chart/ffn.rs:246-252), then
// quantizes it (quant_act) with its block's lanes: act_scale is monotone in the block's largest
// magnitude, so the block exponent is the largest of the lanes' own exponents (a 32-lane max of
// small integers), and each lane forms its own code.  Refusals keep the reference FFN's order
// (chart/ffn.rs:1712-1720): the projections' outputs (recorded by the tile loop, gate rows then
// up rows), then the elements' conversion or SwiGLU refusals, then the quantizer's, each class
// keyed past the one before.
AH_DEV void ffn_epilogue(const FfnArgs &fa, uint32_t b0, uint32_t b1, const float *hsum,
                         unsigned long long *status) {
    ah_lds_barrier();  // every wave's row sums are in LDS
    const uint32_t n = fa.n_ff, nb = (n + 31) / 32;
    const uint32_t tid = threadIdx.x, j = tid / 32, l = tid & 31;
    const uint32_t b = b0 + j, k = 32 * b + l;  // b1 - b0 <= kSThreads / 32
    if (b0 + j >= b1) return;                    // whole half-waves: uniform per 32-lane group
    const bool live = k < n;
    const uint32_t gb = live ? __builtin_bit_cast(uint32_t, hsum[k - 32 * b0]) : 0u;
    const uint32_t ub = live ? __builtin_bit_cast(uint32_t, hsum[kFfnRows + k - 32 * b0]) : 0u;
    // quant_act of the block (chart/mod.rs:258-334): S = act_scale(max |h|), codes q + [2r >= S]
    const HiddenQ q = swiglu_quant32(gb, ub, live);
    if (q.err) ah_record(status, ah_out_key(2ull * n + k, (uint32_t)q.err));
    const __amdgpu_buffer_rsrc_t rc = ah_rsrc(fa.h_codes, n), rs = ah_rsrc(fa.h_scales, nb * 8u);
    __builtin_amdgcn_raw_buffer_store_b8((uint8_t)q.code, rc, live ? k : kActOob, 0, 0);
    if (l == 0) {
        if (q.bad_block) ah_record(status, ah_out_key(3ull * n + b, 7u));
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, (u32x2){(uint32_t)q.scale, (uint32_t)(q.scale >> 32)}),
                                              rs, 8 * b, 0, 0);
    }
}

// The unfused prefill FFN's SwiGLU pass: the gate and up projections' f32 outputs [n_tok][n_ff]
// into the hidden QuantAct, codes [n_tok][n_ff] and scales [n_tok][ceil(n_ff / 32)], as
// swiglu_cols then quant_cols do per column (chart/ffn.rs:493-560, chart/mod.rs:258-334).  One
// 32-lane half-wave per (token, hidden block), the wave's two blocks consecutive; refusals keyed
// past the projections': an element's conversion or SwiGLU at key_sw + t * n_ff + k, a block's
// quantizer at key_q + t * ceil(n_ff / 32) + b.
__global__ void __launch_bounds__(kThreads) swiglu_quant_kernel(SwigluArgs a) {
    const uint32_t nbh = (a.n_ff + 31) / 32;
    const uint64_t total = (uint64_t)a.n_tok * nbh;
    const uint32_t lane = threadIdx.x & 63u, l = lane & 31u, half = lane >> 5;
    const uint64_t wave = ((uint64_t)blockIdx.x * kThreads + threadIdx.x) / 64;
    const uint64_t waves = (uint64_t)gridDim.x * (kThreads / 64);
    for (uint64_t p = wave; 2 * p < total; p += waves) {  // the same trip count for the whole wave
        const uint64_t blk = 2 * p + half;
        const bool vb = blk < total;
        const uint32_t t = vb ? (uint32_t)(blk / nbh) : 0u, b = vb ? (uint32_t)(blk % nbh) : 0u;
        const uint32_t k = 32u * b + l;
        const bool live = vb && k < a.n_ff;
        const size_t e = (size_t)t * a.n_ff + k;
        const uint32_t gb = live ? __builtin_bit_cast(uint32_t, a.gate[e]) : 0u;
        const uint32_t ub = live ? __builtin_bit_cast(uint32_t, a.up[e]) : 0u;
        const HiddenQ q = swiglu_quant32(gb, ub, live);
        if (q.err) ah_record(a.status, ah_out_key(a.key_sw + e, (uint32_t)q.err));
        if (live) a.h_codes[e] = (int8_t)q.code;
        if (vb && l == 0) {
            if (q.bad_block) ah_record(a.status, ah_out_key(a.key_q + blk, 7u));
            a.h_scales[blk] = (int64_t)q.scale;
        }
    }
}

// FFN: the fused FFN's gate/up launch (argument parts 0 = gate, 1 = up; FfnArgs): workgroup w
// serves hidden blocks [w * blocks_per_wg, +blocks_per_wg), waves 0-3 its gate rows and waves 4-7
// its up rows; the row sums also go to LDS, and the SwiGLU epilogue writes the hidden QuantAct.
// (The fused FFN's Q6_K form is built for 2 waves per SIMD: at 4 it spilled 16 bytes a lane.)
template <int TYPE, bool PLAN, bool DOTS, bool FFN = false>
__global__ void __launch_bounds__(kSThreads, FFN && TYPE == AH_GGML_Q6_K ? 2 : stream_waves_per_simd<TYPE>())
    gemv_stream_kernel(StreamParts sp, const GemvPart *__restrict__ parts,
                       const StreamWG *__restrict__ wgd, uint32_t act_bytes,
                       unsigned long long *status, FfnArgs fa) {
    static_assert(!FFN || (!PLAN && !DOTS), "the FFN launch takes argument parts");
    extern __shared__ __align__(16) uint8_t smem[];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
    GemvPart P;
    uint32_t r_begin, r_end, aoff = 0;
    uint32_t f_b0 = 0, f_b1 = 0;  // FFN: the workgroup's hidden blocks
    if constexpr (FFN) {
        // one part's words per wave, read at a uniform index (selecting between both parts'
        // words would hold them all in scalar registers)
        P = sp.p[__builtin_amdgcn_readfirstlane(wv < kSWaves / 2 ? 0u : 1u)];
        const uint32_t nb = (fa.n_ff + 31) / 32;
        f_b0 = blockIdx.x * fa.blocks_per_wg;
        f_b1 = f_b0 + fa.blocks_per_wg < nb ? f_b0 + fa.blocks_per_wg : nb;
        const uint32_t row0 = 32 * f_b0, rows = (32 * f_b1 < fa.n_ff ? 32 * f_b1 : fa.n_ff) - row0;
        const uint32_t qw = wv % (kSWaves / 2);
        r_begin = row0 + rows * qw / (kSWaves / 2);
        r_end = row0 + rows * (qw + 1) / (kSWaves / 2);
    } else if constexpr (PLAN) {
        const StreamWG *D = wgd + blockIdx.x;
        const uint32_t pi = D->wave_part[wv];
        const bool idle = pi == kIdleWave;
        P = part_at(parts, idle ? D->act_part[0] : pi);  // an idle wave streams no rows
        r_begin = D->r_begin[wv];
        r_end = idle ? r_begin : D->r_end[wv];
        aoff = D->act_off[D->wave_act[wv]];
    } else {
        // The workgroup's part.  One round of argument loads brings the part count, the later
        // parts' first workgroups and every word of part 0 (held in scalar registers by the empty
        // asm statements, so the loads go out together); a workgroup of a later part then reads
        // that part's words in a second round, at a uniform offset into the arguments.
        auto pin = [](const GemvPart &q) {
            uint32_t pw[sizeof(GemvPart) / 4];
            __builtin_memcpy(pw, &q, sizeof(GemvPart));
#pragma unroll
            for (uint32_t i = 0; i < sizeof(GemvPart) / 4; ++i) __asm__ volatile("" ::"s"(pw[i]));
        };
        P = sp.p[0];
        const uint32_t np = sp.n, b1 = sp.p[1].wg_begin, b2 = sp.p[2].wg_begin, b3 = sp.p[3].wg_begin;
        __asm__ volatile("" ::"s"(np), "s"(b1), "s"(b2), "s"(b3));
        pin(P);
        const uint32_t pi = (1u < np && blockIdx.x >= b1 ? 1u : 0u) + (2u < np && blockIdx.x >= b2 ? 1u : 0u) +
                            (3u < np && blockIdx.x >= b3 ? 1u : 0u);
        if (pi != 0) {
            P = sp.p[__builtin_amdgcn_readfirstlane(pi)];
            pin(P);
        }
        const uint32_t n_waves = P.wg_count * kSWaves;
        const uint32_t wl = (blockIdx.x - P.wg_begin) * kSWaves + wave;
        r_begin = (uint32_t)((uint64_t)P.n_out * wl / n_waves);
        r_end = (uint32_t)((uint64_t)P.n_out * (wl + 1) / n_waves);
    }
    // GEMV parts take f32 or code inputs (the Q32.32 form is the quantizer's alone): telling the
    // compiler drops that form's 16-word inputs from the prologue's registers
    __builtin_assume(P.src != AH_SRC_Q32);
    const uint32_t kpad = (P.n_in + 255) / 256 * 256;
    const ActLds A = carve(smem + aoff, kpad);
    uint8_t *tl = smem + act_bytes + wave * kSlotBytes;
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(P.w, (uint32_t)P.w_bytes);
    const uint32_t U = P.units, RW = P.rows_per_tile, RB = P.row_bytes, G = P.lanes;
    const uint32_t n_t = (r_end - r_begin + RW - 1) / RW;

    // Tile t's loads.  All kChunks loads are issued, chunks past the tile out of range (they read
    // nothing), so that the compiler's load counting sees the same loads on every path and never
    // waits for one that is still streaming when it only needs an older one.  A wave requests no
    // tile past its last: the out-of-range loads of an empty tile still take the vector memory
    // path (a decode token took 3% longer with them).
    u32x4 chunk[kChunks];
    auto load_tile = [&](uint32_t t) {
        const uint32_t r0 = r_begin + t * RW;
        const uint32_t rows = t >= n_t ? 0u : (r_end - r0 < RW ? r_end - r0 : RW);
        const uint32_t start = rows ? r0 * RB : 0u, a0 = start & ~15u;
        const uint32_t nch = rows ? (rows * RB + (start - a0) + 15) / 16 : 0u;
#pragma unroll
        for (uint32_t i = 0; i < kChunks; ++i) {
            const uint32_t c = lane + 64 * i;
            chunk[i] = ah_ld128_nt(rs, c < nch ? a0 + 16 * c : kOob);
        }
    };

    // Prologue.  Single part: every wave's activation loads go out before any tile load of the
    // workgroup (the barrier orders issue, not completion), tile 0 follows at once, and the
    // quantizer runs from registers while tile 0 streams in.  Plan: each wave requests its own
    // tile 0 first, then the workgroup quantizes its activations one after another.  After the
    // barrier that publishes the activations each wave stages its own tile 0 and requests tile 1,
    // so no wave waits for another's tile.
    constexpr uint32_t QB = kSThreads / 4;
    if constexpr (PLAN) {
        load_tile(0);
        const StreamWG *D = wgd + blockIdx.x;
        const uint32_t n_act = D->n_act;
        for (uint32_t a = 0; a < n_act; ++a) {
            const GemvPart Pa = part_at(parts, D->act_part[a]);
            __builtin_assume(Pa.src != AH_SRC_Q32);
            const uint32_t nbpa = (Pa.n_in + 255) / 256 * 8;
            const ActLds Aa = carve(smem + D->act_off[a], nbpa * 32);
            const ActRsrc xra = act_rsrc(Pa.x, Pa.scales, Pa.src, Pa.n_in);
            for (uint32_t base = 0; base < nbpa; base += QB) {
                if (base + wave * 16 >= nbpa) break;  // this wave's 16 blocks lie past the activation
                const uint32_t b = base + threadIdx.x / 4;
                // (the Q6_K plan kernel sits at its register budget: the integer code form there)
                const QuadOut o = quad_quant(quad_load_row(xra, Pa.src, Pa.n_in, b), Pa.src, b, status, 0,
                                             TYPE != AH_GGML_Q6_K);
                if (b < nbpa) store_quad(Aa, b, o);
            }
        }
    } else {
        const uint32_t nbp = kpad / 32;
        const uint32_t passes = (nbp + QB - 1) / QB;
        const ActRsrc xr = act_rsrc(P.x, P.scales, P.src, P.n_in);
        // (a wave whose blocks of a pass all lie past the activation requests nothing for it: the
        // empty passes' out-of-range loads had cost a decode token 2%)
        QuadIn x0 = {}, x1 = {};
        if (wave * 16 < nbp) x0 = quad_load_row(xr, P.src, P.n_in, threadIdx.x / 4);
        if (QB + wave * 16 < nbp) x1 = quad_load_row(xr, P.src, P.n_in, QB + threadIdx.x / 4);
        ah_lds_barrier();
        load_tile(0);
        // Pass p quantizes blocks p*QB + tid/4.  A wave whose 16 blocks of a pass all lie past the
        // activation has nothing to quantize in it (nor in any later pass).  The third pass's
        // input (K > 8192) is requested once pass 0 has consumed x0, so its load overlaps pass 1.
        const uint32_t b0 = threadIdx.x / 4;
        const bool w0 = wave * 16 < nbp;
        const unsigned long long kb = (unsigned long long)P.key_tok * P.n_in;
        QuadOut o0 = {};
        if (w0) o0 = quad_quant(x0, P.src, b0, status, kb);
        QuadIn x2 = {};
        if (2 * QB + wave * 16 < nbp) x2 = quad_load_row(xr, P.src, P.n_in, 2 * QB + b0);
        if (w0 && b0 < nbp) store_quad(A, b0, o0);
        if (passes > 1 && QB + wave * 16 < nbp) {
            const QuadOut o = quad_quant(x1, P.src, QB + b0, status, kb);
            if (QB + b0 < nbp) store_quad(A, QB + b0, o);
        }
        if (passes > 2 && 2 * QB + wave * 16 < nbp) {
            const QuadOut o = quad_quant(x2, P.src, 2 * QB + b0, status, kb);
            if (2 * QB + b0 < nbp) store_quad(A, 2 * QB + b0, o);
        }
        // activations past 3 * 128 blocks (K > 12288); Q6_K keeps the general form here, as the
        // fast one's temporaries in this loop push its tile loop's allocation into spills
        for (uint32_t p = 3; p < passes; ++p) {
            const uint32_t b = p * QB + b0;
            if (p * QB + wave * 16 >= nbp) break;
            const QuadOut o = quad_quant(quad_load_row(xr, P.src, P.n_in, b), P.src, b, status, kb,
                                         TYPE != AH_GGML_Q6_K);
            if (b < nbp) store_quad(A, b, o);
        }
    }
    auto stage = [&](uint32_t t) {  // tile t (in registers) to the slot; request tile t + 1
#pragma unroll
        for (uint32_t i = 0; i < kChunks; ++i) reinterpret_cast<u32x4 *>(tl)[lane + 64 * i] = chunk[i];
        if (t + 1 < n_t) load_tile(t + 1);
    };
    ah_lds_barrier();  // the activation is published; tiles are wave-private, so each wave
    stage(0);          // stages its own tile 0 (unconditionally: a wave without rows stages zeros)

    // Row sums leave through a buffer store that every lane issues (lanes that own no row store
    // out of range, which writes nothing): a store behind a branch would make the compiler wait for
    // its completion before the next tile is staged.
    const __amdgpu_buffer_rsrc_t ry = ah_rsrc(P.y, P.y ? P.n_out * 4u : 0u);  // FFN: y optional
    float *const hsum = reinterpret_cast<float *>(smem + act_bytes + kSWaves * kSlotBytes);
    const uint32_t r = lane / G, g = lane & (G - 1);
    // earliest refused output row of the wave, (row << 1) | (code == 9), kept in a scalar register
    // (a ballot, no memory operation in the loop); recorded once after the last tile
    uint32_t obad = 0xFFFFFFFFu;
    for (uint32_t t = 0; t < n_t; ++t) {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS stores have landed
        __builtin_amdgcn_wave_barrier();
        const uint32_t r0 = r_begin + t * RW;
        const uint32_t toff = (r0 * RB) & 15u;
        const uint32_t row = r0 + r;
        const bool owns = r < RW && row < r_end;
        float acc = 0.0f;
        if (owns) {
            if constexpr (TYPE == kMixedType) {
                if (P.type == AH_GGML_Q4_K) {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q4_K, DOTS, !PLAN>(P, tl, toff + r * RB, row, u, A);
                } else if (P.type == AH_GGML_Q6_K) {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q6_K, DOTS, !PLAN>(P, tl, toff + r * RB, row, u, A);
                } else if (P.type == AH_GGML_Q5_0) {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q5_0, DOTS, !PLAN>(P, tl, toff + r * RB, row, u, A);
                } else if (P.type == AH_GGML_Q2_K) {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q2_K, DOTS, !PLAN>(P, tl, toff + r * RB, row, u, A);
                } else if (P.type == AH_GGML_Q3_K) {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q3_K, DOTS, !PLAN>(P, tl, toff + r * RB, row, u, A);
                } else {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q8_0, DOTS, !PLAN>(P, tl, toff + r * RB, row, u, A);
                }
            } else {
#pragma unroll 1
                for (uint32_t u = g; u < U; u += G)
                    acc += comp_unit<TYPE, DOTS, !PLAN>(P, tl, toff + r * RB, row, u, A);
            }
        }
        acc = group_sum(acc, G);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc), ry,
                                              (g == G - 1 && owns) ? row * 4u : kOob, 0, 0);
        if constexpr (FFN)
            if (g == G - 1 && owns) hsum[(wv < kSWaves / 2 ? 0u : kFfnRows) + row - 32 * f_b0] = acc;
        const uint32_t oc = ah_out_code(acc);
        const uint64_t ob = __builtin_amdgcn_ballot_w64(g == G - 1 && owns && oc != 0u);
        if (ob) {  // uniform: lanes own rows in lane order, so the lowest lane is the earliest row
            const uint32_t k = __builtin_amdgcn_readlane((row << 1) | (oc == 9u ? 1u : 0u), (int)__builtin_ctzll(ob));
            obad = k < obad ? k : obad;
        }
        __builtin_amdgcn_wave_barrier();  // all lanes are done reading the slot before it is refilled
        if (t + 1 < n_t) stage(t + 1);    // (past the last tile nothing is staged: no wait for its loads)
    }
    if constexpr (FFN) {
        // gate rows keep their index, up rows follow them (the reference projects gate, then up)
        if (obad != 0xFFFFFFFFu && lane == 0)
            ah_record(status, ah_out_key((obad >> 1) + (wv < kSWaves / 2 ? 0u : fa.n_ff), (obad & 1u) ? 9u : 8u));
        ffn_epilogue(fa, f_b0, f_b1, hsum, status);
    } else {
        if (obad != 0xFFFFFFFFu && lane == 0)
            ah_record(status, ah_out_key(P.out_key0 + (obad >> 1), (obad & 1u) ? 9u : 8u));
    }
}

// ---- persistent decode sequence ---------------------------------------------------------------
//
// A token's projections form a chain of stages (q/k/v -> o -> gate/up -> SwiGLU -> down per layer,
// then the head): each stage reads an earlier stage's output.  One kernel launch per stage pays a
// dispatch, the grid's fill and the activation prologue in series for every stage.  Here one
// resident grid runs the whole chain as a dataflow: a workgroup takes part in a stage only if the
// stage's plan gives it work; when its outputs are stored (device-scope sc1 stores, complete before
// it signals) it counts itself into its group's completion counter for that stage.  A workgroup
// with work in stage s+1 first requests its weight tiles (they do not depend on stage s), then
// waits until every group counter of stage s has reached this launch's target (run number x the
// group's producers), then reads stage s's outputs (sc1 loads).  Waiting for stage s implies every
// earlier stage (each producer of s waited for s-1), so stages cannot overtake one another, and no
// workgroup rewrites a buffer an earlier stage still reads.  Workgroups idle in a stage skip it.
//
// Counters: one per group of kSeqGroup workgroups and stage, each on its own 128-byte line, so a
// stage's increments spread over up to kSeqMaxGroups addresses (one counter for a whole 512-wide
// grid serializes its atomics: 7.2 us a barrier measured, against 2.7 us for groups of 16-32).
// Lane g of wave 0 polls group g's counter, so one load instruction checks every group; polls are
// bounded (past spin_limit the stage records AH_ERR_SEQ_TIMEOUT and waits no more in this launch).
// A workgroup's run number is its own device counter, read at start and bumped at the end.  The
// grid is at most what the device holds at once (see ah_launch_gemv_seq).

// The SwiGLU stage: the hidden activation's 32-blocks are dealt to the workgroups, 16 blocks per
// round (one element per thread): gate and up from f32 to Q32.32 (to_q32), h = swiglu into LDS,
// then a quad of lanes per block quantizes it (quant_act) into the hidden QuantAct the down stage
// reads.  Refusals in element order (conversion or SwiGLU), then the quantizer's, as the
// reference FFN orders them (chart/ffn.rs:1712-1720).  `hl` is 512 int64 of LDS.
AH_DEV void swiglu_stage(const SeqStage &S, unsigned long long *st, int64_t *hl) {
    constexpr uint32_t kRound = kSThreads / 32;  // blocks per round
    const uint32_t nb = (S.n + 31) / 32;
    const uint32_t b0 = (uint32_t)((uint64_t)nb * blockIdx.x / gridDim.x);
    const uint32_t b1 = (uint32_t)((uint64_t)nb * (blockIdx.x + 1) / gridDim.x);
    const __amdgpu_buffer_rsrc_t rg = ah_rsrc(S.gate, S.n * 4u), ru = ah_rsrc(S.up, S.n * 4u);
    const __amdgpu_buffer_rsrc_t rc = ah_rsrc(S.codes, S.n), rs = ah_rsrc(S.scales, nb * 8u);
    const uint32_t q = threadIdx.x & 3;
    for (uint32_t base = b0; base < b1; base += kRound) {  // a uniform trip count
        const uint32_t k = 32 * base + threadIdx.x;
        const bool live = k < 32 * b1 && k < S.n;
        const uint32_t gb = __builtin_amdgcn_raw_buffer_load_b32(rg, live ? 4 * k : kActOob, 0, kCoherent);
        const uint32_t ub = __builtin_amdgcn_raw_buffer_load_b32(ru, live ? 4 * k : kActOob, 0, kCoherent);
        int64_t h = 0;
        if (live) {
            uint64_t mg, mu;
            bool ng, nu;
            int e = ah_to_q32_mag(gb, mg, ng);
            if (!e) e = ah_to_q32_mag(ub, mu, nu);
            if (!e) e = swiglu_fx(ng ? (int64_t)(0ull - mg) : (int64_t)mg, nu ? (int64_t)(0ull - mu) : (int64_t)mu, h);
            if (e) {
                ah_record(st, ((unsigned long long)k << 8) | (unsigned)e);
                h = 0;
            }
        }
        hl[threadIdx.x] = h;
        ah_lds_barrier();
        // quads: lane q of the quad for block base + j (j < 16, 4 * 16 = 64 lanes of wave 0 .. 1)
        if (threadIdx.x < 4 * kRound) {
            const uint32_t j = threadIdx.x / 4, b = base + j, k0 = 32 * b + 8 * q;
            QuadIn in;
            in.take = b < b1 && S.n > k0 ? (S.n - k0 < 8 ? S.n - k0 : 8) : 0;
            in.s0 = in.s1 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint64_t v = (uint32_t)i < in.take ? (uint64_t)hl[32 * j + 8 * q + i] : 0ull;
                in.w[2 * i] = (uint32_t)v;
                in.w[2 * i + 1] = (uint32_t)(v >> 32);
            }
            const QuadOut o = quad_quant(in, AH_SRC_Q32, b, st, 0);
            if (b < b1) {
                if (in.take == 8) {
                    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, (u32x2){o.c0, o.c1}), rc, k0, 0, kCoherent);
                } else {
#pragma unroll
                    for (uint32_t i = 0; i < 8; ++i)
                        if (i < in.take)
                            __builtin_amdgcn_raw_buffer_store_b8((uint8_t)(((i < 4 ? o.c0 : o.c1) >> (8 * (i & 3))) & 0xffu), rc,
                                                                 k0 + i, 0, kCoherent);
                }
                if (q == 0) {
                    const uint64_t S64 = o.e < 0 ? 0ull : (1ull << o.e);
                    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, (u32x2){(uint32_t)S64, (uint32_t)(S64 >> 32)}),
                                                          rs, 8 * b, 0, kCoherent);
                }
            }
        }
        ah_lds_barrier();  // hl is reused by the next round
    }
}

// Wave 0 of a workgroup waits until stage `sp`'s counters reach run r's targets.
AH_DEV void seq_wait(const SeqArgs &a, uint32_t sp, uint32_t r, unsigned long long *st, bool &broken) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t ngrp = (gridDim.x + kSeqGroup - 1) / kSeqGroup;
    const uint32_t need = lane < ngrp ? a.producers[a.stages[sp].prod_off + lane] * r : 0u;
    const unsigned *cnt = a.done + (size_t)(sp * kSeqMaxGroups + (lane < ngrp ? lane : 0)) * kSeqLine;
    uint32_t polls = 0;
    while (!broken) {
        const unsigned v = lane < ngrp ? __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
        if (__builtin_amdgcn_ballot_w64(v < need) == 0) break;
        if (++polls >= a.spin_limit) {  // every later wait of this launch is skipped
            if (lane == 0) ah_record(st, kSeqTimeoutKey);
            broken = true;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
}
// Thread 0 counts the workgroup into stage s's group counter (after every wave's stores are done).
AH_DEV void seq_signal(const SeqArgs &a, uint32_t s) {
    if (threadIdx.x == 0)
        (void)__hip_atomic_fetch_add(a.done + (size_t)(s * kSeqMaxGroups + blockIdx.x / kSeqGroup) * kSeqLine, 1u,
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One GEMV stage of the sequence: the workgroup's waves stream their rows of the stage's parts
// (the PLAN form of gemv_stream_kernel) with device-scope output stores.
template <int TYPE>
AH_DEV void seq_gemv_stage(const SeqArgs &a, uint32_t s, uint32_t r, bool &broken) {
    extern __shared__ __align__(16) uint8_t smem[];
    const SeqStage &S = a.stages[s];
    const StreamWG *D = a.wgd + S.wgd_off + blockIdx.x;
    const uint32_t n_act = D->n_act;
    if (n_act == 0) return;  // no work for this workgroup in this stage
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
    uint8_t *tl = smem + a.act_bytes + wave * kSlotBytes;
    constexpr uint32_t QB = kSThreads / 4;
    unsigned long long *st = a.status + s;
    const uint32_t pi = D->wave_part[wv];
    const bool idle = pi == kIdleWave;
    const GemvPart P = part_at(a.parts, idle ? D->act_part[0] : pi);  // an idle wave streams no rows
    const uint32_t r_begin = D->r_begin[wv], r_end = idle ? r_begin : D->r_end[wv];
    const ActLds A = carve(smem + D->act_off[D->wave_act[wv]], (P.n_in + 255) / 256 * 256);
    const __amdgpu_buffer_rsrc_t rsw = ah_rsrc(P.w, (uint32_t)P.w_bytes);
    const uint32_t U = P.units, RW = P.rows_per_tile, RB = P.row_bytes, G = P.lanes;
    const uint32_t n_t = (r_end - r_begin + RW - 1) / RW;
    u32x4 chunk[kChunks];
    auto load_tile = [&](uint32_t t) {
        const uint32_t r0 = r_begin + t * RW;
        const uint32_t rows = t >= n_t ? 0u : (r_end - r0 < RW ? r_end - r0 : RW);
        const uint32_t start = rows ? r0 * RB : 0u, a0 = start & ~15u;
        const uint32_t nch = rows ? (rows * RB + (start - a0) + 15) / 16 : 0u;
#pragma unroll
        for (uint32_t i = 0; i < kChunks; ++i) {
            const uint32_t c = lane + 64 * i;
            chunk[i] = ah_ld128_nt(rsw, c < nch ? a0 + 16 * c : kOob);
        }
    };
    // Weights do not depend on the previous stage: waves 1-7 request their tile 0 at once; wave 0
    // first waits for the previous stage (its loads would hold up its polls: vector memory
    // operations complete in order), then requests its own.
    ah_lds_barrier();  // the previous stage's LDS readers are done
    if (s) {
        if (wv != 0) load_tile(0);
        else seq_wait(a, s - 1, r, st, broken);
        ah_lds_barrier();
        if (wv == 0) load_tile(0);
    } else {
        load_tile(0);
    }
    for (uint32_t ai = 0; ai < n_act; ++ai) {
        const GemvPart Pa = part_at(a.parts, D->act_part[ai]);
        const uint32_t nbpa = (Pa.n_in + 255) / 256 * 8;
        const ActLds Aa = carve(smem + D->act_off[ai], nbpa * 32);
        const ActRsrc xra = act_rsrc(Pa.x, Pa.scales, Pa.src, Pa.n_in);
        for (uint32_t base = 0; base < nbpa; base += QB) {
            if (base + wave * 16 >= nbpa) break;
            const uint32_t b = base + threadIdx.x / 4;
            const QuadOut o = quad_quant(quad_load_row<kCoherent>(xra, Pa.src, Pa.n_in, b), Pa.src, b, st, 0);
            if (b < nbpa) store_quad(Aa, b, o);
        }
    }
    auto stage = [&](uint32_t t) {
#pragma unroll
        for (uint32_t i = 0; i < kChunks; ++i) reinterpret_cast<u32x4 *>(tl)[lane + 64 * i] = chunk[i];
        if (t + 1 < n_t) load_tile(t + 1);
    };
    ah_lds_barrier();
    stage(0);
    const __amdgpu_buffer_rsrc_t ry = ah_rsrc(P.y, P.n_out * 4u);
    const uint32_t rr = lane / G, g = lane & (G - 1);
    uint32_t obad = 0xFFFFFFFFu;
    for (uint32_t t = 0; t < n_t; ++t) {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS stores have landed
        __builtin_amdgcn_wave_barrier();
        const uint32_t r0 = r_begin + t * RW;
        const uint32_t toff = (r0 * RB) & 15u;
        const uint32_t row = r0 + rr;
        const bool owns = rr < RW && row < r_end;
        float acc = 0.0f;
        if (owns) {
            if constexpr (TYPE == kMixedType) {
                if (P.type == AH_GGML_Q4_K) {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q4_K, false, true>(P, tl, toff + rr * RB, row, u, A);
                } else if (P.type == AH_GGML_Q6_K) {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q6_K, false, true>(P, tl, toff + rr * RB, row, u, A);
                } else if (P.type == AH_GGML_Q5_0) {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q5_0, false, true>(P, tl, toff + rr * RB, row, u, A);
                } else if (P.type == AH_GGML_Q2_K) {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q2_K, false, true>(P, tl, toff + rr * RB, row, u, A);
                } else if (P.type == AH_GGML_Q3_K) {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q3_K, false, true>(P, tl, toff + rr * RB, row, u, A);
                } else {
#pragma unroll 1
                    for (uint32_t u = g; u < U; u += G)
                        acc += comp_unit<AH_GGML_Q8_0, false, true>(P, tl, toff + rr * RB, row, u, A);
                }
            } else {
#pragma unroll 1
                for (uint32_t u = g; u < U; u += G)
                    acc += comp_unit<TYPE, false, true>(P, tl, toff + rr * RB, row, u, A);
            }
        }
        acc = group_sum(acc, G);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc), ry,
                                              (g == G - 1 && owns) ? row * 4u : kOob, 0, kCoherent);
        const uint32_t oc = ah_out_code(acc);
        const uint64_t ob = __builtin_amdgcn_ballot_w64(g == G - 1 && owns && oc != 0u);
        if (ob) {
            const uint32_t k = __builtin_amdgcn_readlane((row << 1) | (oc == 9u ? 1u : 0u), (int)__builtin_ctzll(ob));
            obad = k < obad ? k : obad;
        }
        __builtin_amdgcn_wave_barrier();
        if (t + 1 < n_t) stage(t + 1);
    }
    if (obad != 0xFFFFFFFFu && lane == 0) ah_record(st, ah_out_key(obad >> 1, (obad & 1u) ? 9u : 8u));
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's outputs are complete
    ah_lds_barrier();
    seq_signal(a, s);
}

AH_DEV void seq_swiglu_stage(const SeqArgs &a, uint32_t s, uint32_t r, bool &broken) {
    extern __shared__ __align__(16) uint8_t smem[];
    const SeqStage &S = a.stages[s];
    const uint32_t nb = (S.n + 31) / 32;
    if ((uint64_t)nb * blockIdx.x / gridDim.x == (uint64_t)nb * (blockIdx.x + 1) / gridDim.x) return;  // no blocks
    unsigned long long *st = a.status + s;
    ah_lds_barrier();
    if (s && __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) == 0) seq_wait(a, s - 1, r, st, broken);
    ah_lds_barrier();
    swiglu_stage(S, st, reinterpret_cast<int64_t *>(smem));
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    ah_lds_barrier();
    seq_signal(a, s);
}

// Built for 2 waves per SIMD (one resident workgroup per CU, <= 256 VGPRs): at 4 the Q4_K and
// Q6_K forms spilled ~100 bytes a lane, and the configs[4] token measured the same either way
// (827-829 us).
template <int TYPE>
__global__ void __launch_bounds__(kSThreads, 2) gemv_seq_kernel(SeqArgs a) {
    // this launch's run number (nothing writes the counter until the workgroup ends)
    const uint32_t r = __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(a.runs + blockIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1);
    bool broken = false;  // (wave 0) a wait timed out: the launch's results are refused
    for (uint32_t s = 0; s < a.n_stages; ++s) {
        if (a.stages[s].kind == kSeqSwiglu) seq_swiglu_stage(a, s, r, broken);
        else seq_gemv_stage<TYPE>(a, s, r, broken);
    }
    if (threadIdx.x == 0) __hip_atomic_store(a.runs + blockIdx.x, r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Stream geometry for a row of RB bytes and U units: whole rows per tile and lanes per row.
// Returns false when a row does not fit one tile (the workgroup-tile kernel then serves the part).
// A lane computes ceil(units / G) units of its row per tile, so (rows, G) is chosen for the most
// row bytes per round of unit work (ties to more rows): e.g. Q4_K at K = 1536 takes 8 rows of 8
// lanes (one super-block each) rather than 9 rows of 4 (two each).
// Rows per wave tile and lanes per row of a streaming part.  Whole-unit parts (32-blocks, Q4_K
// super-blocks, Q6_K halves) maximize the bytes a wave streams per round of units (measured best
// for them at every decode and batch shape).  Q4_K pair units (chosen for small projections, see
// units_per_row's callers) minimize a wave's time instead: tiles per wave times the rounds of pairs
// per tile plus the tile's fixed steps (staging, the row sums, the store: about two pairs), over a
// device of kLatencyWaves waves, so a small projection spreads over many waves with one round each.
// Ties go to more rows per tile (fewer workgroups).  The choice depends on the part alone.
bool ah_gemv_stream_geometry(uint32_t type, uint32_t row_bytes, uint32_t units, uint32_t n_out, uint32_t &rows,
                             uint32_t &lanes) {
    if (row_bytes == 0 || row_bytes + 16 > kStreamTile) return false;
    const uint32_t fit = (kStreamTile - 16) / row_bytes;
    const bool pairs = type == AH_GGML_Q4_K && row_bytes / (units ? units : 1u) < 64;
    rows = 1;
    lanes = 64;
    if (!pairs) {
        uint64_t best = 0;
        for (uint32_t G = 1; G <= 64; G <<= 1) {
            const uint32_t r = fit < 64 / G ? fit : 64 / G;
            const uint32_t rounds = units > G ? (units + G - 1) / G : 1u;
            const uint64_t score = (uint64_t)r * row_bytes * 64 / rounds;
            if (score > best) {
                best = score;
                rows = r;
                lanes = G;
            }
        }
        return true;
    }
    constexpr uint64_t kLatencyWaves = 2048;  // 8 waves on each of 256 CUs
    uint64_t best = ~0ull;
    for (uint32_t G = 1; G <= 64; G <<= 1) {
        const uint32_t r = fit < 64 / G ? fit : 64 / G;
        const uint64_t rounds = units > G ? (units + G - 1) / G : 1u;
        const uint64_t tiles = (n_out + r - 1) / r;
        const uint64_t per_wave = (tiles + kLatencyWaves - 1) / kLatencyWaves;
        const uint64_t cost = per_wave * (rounds + 2);
        if (cost < best || (cost == best && r > rows)) {
            best = cost;
            rows = r;
            lanes = G;
        }
    }
    return true;
}

// LDS bytes of one part's quantized activation (codes with padding, fsc, xs32, xs16): a multiple
// of 16 for any kpad that is a multiple of 256.
size_t ah_gemv_act_bytes(uint32_t kpad) {
    return kpad + kpad / 16 + (size_t)kpad / 32 * 8 + (size_t)kpad / 16 * 4;
}
size_t ah_gemv_stream_slot_bytes() { return (size_t)kSWaves * kSlotBytes; }
size_t ah_gemv_stream_lds_bytes(uint32_t kpad_max) { return ah_gemv_act_bytes(kpad_max) + ah_gemv_stream_slot_bytes(); }

uint32_t ah_gemv_stream_threads() { return kSThreads; }

static const void *stream_fn(uint32_t type, bool plan, bool dots = false) {
#define AH_SFN(T) return plan ? reinterpret_cast<const void *>(&gemv_stream_kernel<T, true, false>)     \
                      : dots ? reinterpret_cast<const void *>(&gemv_stream_kernel<T, false, true>)     \
                             : reinterpret_cast<const void *>(&gemv_stream_kernel<T, false, false>);
    if (type == kMixedType)  // a table plan or argument parts (no debug form)
        return plan ? reinterpret_cast<const void *>(&gemv_stream_kernel<kMixedType, true, false>)
                    : dots ? nullptr : reinterpret_cast<const void *>(&gemv_stream_kernel<kMixedType, false, false>);
    switch (type) {
    case AH_GGML_Q8_0: AH_SFN(AH_GGML_Q8_0)
    case AH_GGML_Q5_0: AH_SFN(AH_GGML_Q5_0)
    case AH_GGML_Q2_K: AH_SFN(AH_GGML_Q2_K)
    case AH_GGML_Q3_K: AH_SFN(AH_GGML_Q3_K)
    case AH_GGML_Q4_K: AH_SFN(AH_GGML_Q4_K)
    case AH_GGML_Q6_K: AH_SFN(AH_GGML_Q6_K)
    default: return nullptr;
    }
#undef AH_SFN
}

static const void *seq_fn(uint32_t type) {
    switch (type) {
    case kMixedType: return reinterpret_cast<const void *>(&gemv_seq_kernel<kMixedType>);
    case AH_GGML_Q8_0: return reinterpret_cast<const void *>(&gemv_seq_kernel<AH_GGML_Q8_0>);
    case AH_GGML_Q5_0:  // rare families: no own form
    case AH_GGML_Q2_K:
    case AH_GGML_Q3_K: return reinterpret_cast<const void *>(&gemv_seq_kernel<kMixedType>);
    case AH_GGML_Q4_K: return reinterpret_cast<const void *>(&gemv_seq_kernel<AH_GGML_Q4_K>);
    case AH_GGML_Q6_K: return reinterpret_cast<const void *>(&gemv_seq_kernel<AH_GGML_Q6_K>);
    default: return nullptr;
    }
}

// Workgroups of the sequence kernel that fit one CU at once with `act_bytes` of activation LDS.
int ah_gemv_seq_occupancy(uint32_t type, size_t act_bytes) {
    int n = 0;
    const void *f = seq_fn(type);
    if (!f || hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, kSThreads, act_bytes + ah_gemv_stream_slot_bytes()) != hipSuccess)
        return 0;
    return n;
}

// One launch runs the whole sequence, its grid at most the workgroups the device holds at once
// (ah_gemv_seq_occupancy per CU), so on a device the launch has to itself every workgroup is
// resident, as the grid barriers between stages need.  An ordinary launch, not a cooperative one:
// it measured 2% faster on the configs[4] token (817 against 835 us), and rocprofv3's kernel trace
// of a process that made cooperative launches ended in a segmentation fault at exit, before it
// wrote its results, while the same trace with ordinary launches completes.  Should other work
// hold CUs so that some workgroups start late, the waits are bounded: the run then reports
// AH_ERR_SEQ_TIMEOUT instead of hanging.
hipError_t ah_launch_gemv_seq(uint32_t type, const SeqArgs &a, uint32_t grid, hipStream_t stream) {
    const void *f = seq_fn(type);
    if (!f) return hipErrorInvalidValue;
    SeqArgs arg = a;
    void *args[] = {&arg};
    return hipLaunchKernel(f, dim3(grid), dim3(kSThreads), args,
                           (unsigned)(a.act_bytes + ah_gemv_stream_slot_bytes()), stream);
}

// Workgroups of the streaming kernel that fit one CU at once with `lds` bytes of LDS each
// (type kMixedType: the mixed-type plan kernel).
int ah_gemv_stream_occupancy(uint32_t type, size_t lds) {
    int n0 = 0, n1 = 0;
    const void *f1 = stream_fn(type, true);
    const void *f0 = stream_fn(type, false);
    if (!f0 || hipOccupancyMaxActiveBlocksPerMultiprocessor(&n0, f0, kSThreads, lds) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n1, f1, kSThreads, lds) != hipSuccess) return 0;
    return n0 < n1 ? n0 : n1;
}

// act_bytes: the activation region (a plan's budget; for argument parts ah_gemv_act_bytes of the
// largest kpad).  d_parts: a plan with a workgroup table, else the parts in `sp`.
hipError_t ah_launch_gemv_stream(uint32_t type, const StreamParts &sp, const GemvPart *d_parts,
                                 const StreamWG *d_wgd, uint32_t grid, uint32_t act_bytes,
                                 unsigned long long *status, hipStream_t stream) {
    const size_t lds = act_bytes + ah_gemv_stream_slot_bytes();
#define AH_SLAUNCH(T)                                                                              \
    if (d_parts)                                                                                   \
        hipLaunchKernelGGL((gemv_stream_kernel<T, true, false>), dim3(grid), dim3(kSThreads), lds,  \
                           stream, sp, d_parts, d_wgd, act_bytes, status, FfnArgs{});             \
    else if (sp.p[0].dots)                                                                         \
        hipLaunchKernelGGL((gemv_stream_kernel<T, false, true>), dim3(grid), dim3(kSThreads), lds,  \
                           stream, sp, d_parts, d_wgd, act_bytes, status, FfnArgs{});             \
    else                                                                                           \
        hipLaunchKernelGGL((gemv_stream_kernel<T, false, false>), dim3(grid), dim3(kSThreads), lds, \
                           stream, sp, d_parts, d_wgd, act_bytes, status, FfnArgs{});
    switch (type) {
    case AH_GGML_Q8_0: AH_SLAUNCH(AH_GGML_Q8_0) break;
    case AH_GGML_Q5_0: AH_SLAUNCH(AH_GGML_Q5_0) break;
    case AH_GGML_Q2_K: AH_SLAUNCH(AH_GGML_Q2_K) break;
    case AH_GGML_Q3_K: AH_SLAUNCH(AH_GGML_Q3_K) break;
    case AH_GGML_Q4_K: AH_SLAUNCH(AH_GGML_Q4_K) break;
    case AH_GGML_Q6_K: AH_SLAUNCH(AH_GGML_Q6_K) break;
    case kMixedType:
        if (d_parts)
            hipLaunchKernelGGL((gemv_stream_kernel<kMixedType, true, false>), dim3(grid), dim3(kSThreads), lds,
                               stream, sp, d_parts, d_wgd, act_bytes, status, FfnArgs{});
        else
            hipLaunchKernelGGL((gemv_stream_kernel<kMixedType, false, false>), dim3(grid), dim3(kSThreads), lds,
                               stream, sp, d_parts, d_wgd, act_bytes, status, FfnArgs{});
        break;
    default: return hipErrorInvalidValue;
    }
#undef AH_SLAUNCH
    return hipGetLastError();
}

// The fused FFN's gate/up launch: one workgroup per `fa.blocks_per_wg` hidden blocks (no
// residency requirement: workgroups do not wait for one another).
static const void *ffn_fn(uint32_t type) {
    switch (type) {
    case AH_GGML_Q8_0: return reinterpret_cast<const void *>(&gemv_stream_kernel<AH_GGML_Q8_0, false, false, true>);
    case AH_GGML_Q5_0: return reinterpret_cast<const void *>(&gemv_stream_kernel<AH_GGML_Q5_0, false, false, true>);
    case AH_GGML_Q2_K: return reinterpret_cast<const void *>(&gemv_stream_kernel<AH_GGML_Q2_K, false, false, true>);
    case AH_GGML_Q3_K: return reinterpret_cast<const void *>(&gemv_stream_kernel<AH_GGML_Q3_K, false, false, true>);
    case AH_GGML_Q4_K: return reinterpret_cast<const void *>(&gemv_stream_kernel<AH_GGML_Q4_K, false, false, true>);
    case AH_GGML_Q6_K: return reinterpret_cast<const void *>(&gemv_stream_kernel<AH_GGML_Q6_K, false, false, true>);
    default: return nullptr;
    }
}

size_t ah_ffn_lds_bytes(uint32_t kpad) { return ah_gemv_stream_lds_bytes(kpad) + kFfnLdsBytes; }

// Workgroups of the FFN gate/up kernel that fit one CU at once (its grid is sized to them).
int ah_ffn_occupancy(uint32_t type, uint32_t kpad) {
    int n = 0;
    const void *f = ffn_fn(type);
    if (!f || hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, kSThreads, ah_ffn_lds_bytes(kpad)) != hipSuccess)
        return 0;
    return n;
}

hipError_t ah_launch_ffn_gate_up(uint32_t type, const StreamParts &sp, const FfnArgs &fa, uint32_t grid,
                                 uint32_t act_bytes, unsigned long long *status, hipStream_t stream) {
    if (!ffn_fn(type) || fa.blocks_per_wg == 0 || fa.blocks_per_wg > kFfnMaxBlocks) return hipErrorInvalidValue;
    const size_t lds = act_bytes + ah_gemv_stream_slot_bytes() + kFfnLdsBytes;
    switch (type) {
    case AH_GGML_Q8_0:
        hipLaunchKernelGGL((gemv_stream_kernel<AH_GGML_Q8_0, false, false, true>), dim3(grid), dim3(kSThreads), lds,
                           stream, sp, nullptr, nullptr, act_bytes, status, fa);
        break;
    case AH_GGML_Q5_0:
        hipLaunchKernelGGL((gemv_stream_kernel<AH_GGML_Q5_0, false, false, true>), dim3(grid), dim3(kSThreads), lds,
                           stream, sp, nullptr, nullptr, act_bytes, status, fa);
        break;
    case AH_GGML_Q2_K:
        hipLaunchKernelGGL((gemv_stream_kernel<AH_GGML_Q2_K, false, false, true>), dim3(grid), dim3(kSThreads), lds,
                           stream, sp, nullptr, nullptr, act_bytes, status, fa);
        break;
    case AH_GGML_Q3_K:
        hipLaunchKernelGGL((gemv_stream_kernel<AH_GGML_Q3_K, false, false, true>), dim3(grid), dim3(kSThreads), lds,
                           stream, sp, nullptr, nullptr, act_bytes, status, fa);
        break;
    case AH_GGML_Q4_K:
        hipLaunchKernelGGL((gemv_stream_kernel<AH_GGML_Q4_K, false, false, true>), dim3(grid), dim3(kSThreads), lds,
                           stream, sp, nullptr, nullptr, act_bytes, status, fa);
        break;
    default:
        hipLaunchKernelGGL((gemv_stream_kernel<AH_GGML_Q6_K, false, false, true>), dim3(grid), dim3(kSThreads), lds,
                           stream, sp, nullptr, nullptr, act_bytes, status, fa);
        break;
    }
    return hipGetLastError();
}

// Chunks of 16 bytes per thread per tile: a tile holds whole rows, so rows longer than 16 KB
// need the larger instantiations.
uint32_t ah_gemv_nc(uint32_t row_bytes) {
    const uint32_t need = row_bytes + 16;
    return need <= 4 * 4096 ? 4u : need <= 8 * 4096 ? 8u : 12u;
}

// Whole rows per tile for a part: as many as fit the chunk budget, capped so the tile's units fit
// the LDS partial slots.
uint32_t ah_gemv_rows_per_tile(uint32_t row_bytes, uint32_t units) {
    const uint32_t nc = ah_gemv_nc(row_bytes);
    uint32_t R = (nc * 4096 - 16) / (row_bytes ? row_bytes : 1);
    if (R < 1) R = 1;
    if (units && R * units > kRedSlots) R = kRedSlots / units > 0 ? kRedSlots / units : 1;
    return R;
}

size_t ah_gemv_lds_bytes(uint32_t nc, uint32_t kpad_max) {
    return kpad_max + kpad_max / 16 + (size_t)kpad_max / 32 * 8 + (size_t)kpad_max / 16 * 4 + kRedSlots * 4 +
           (size_t)nc * 4096 + kTileSlack;
}

template <int TYPE>
static void launch_type(uint32_t nc, dim3 grid, size_t lds, hipStream_t stream, const GemvPart &single,
                        const GemvPart *d_parts, const uint32_t *d_wg_part, uint32_t kpad_max,
                        unsigned long long *status) {
    if (nc <= 4)
        hipLaunchKernelGGL((gemv_kernel<TYPE, 4>), grid, dim3(kThreads), lds, stream, single, d_parts,
                           d_wg_part, kpad_max, status);
    else if (nc <= 8)
        hipLaunchKernelGGL((gemv_kernel<TYPE, 8>), grid, dim3(kThreads), lds, stream, single, d_parts,
                           d_wg_part, kpad_max, status);
    else
        hipLaunchKernelGGL((gemv_kernel<TYPE, 12>), grid, dim3(kThreads), lds, stream, single, d_parts,
                           d_wg_part, kpad_max, status);
}

// Allow the large-row instantiations more than 64 KB of dynamic LDS (once per context).
hipError_t ah_gemv_init_attrs() {
    const int lim = 160 * 1024;
    hipError_t e = hipSuccess;
#define AH_ATTR(T, N)                                                                              \
    if (e == hipSuccess)                                                                           \
        e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_kernel<T, N>),                \
                                hipFuncAttributeMaxDynamicSharedMemorySize, lim);
    AH_ATTR(AH_GGML_Q8_0, 4) AH_ATTR(AH_GGML_Q8_0, 8) AH_ATTR(AH_GGML_Q8_0, 12)
    AH_ATTR(AH_GGML_Q5_0, 4) AH_ATTR(AH_GGML_Q5_0, 8) AH_ATTR(AH_GGML_Q5_0, 12)
    AH_ATTR(AH_GGML_Q2_K, 4) AH_ATTR(AH_GGML_Q2_K, 8) AH_ATTR(AH_GGML_Q2_K, 12)
    AH_ATTR(AH_GGML_Q3_K, 4) AH_ATTR(AH_GGML_Q3_K, 8) AH_ATTR(AH_GGML_Q3_K, 12)
    AH_ATTR(AH_GGML_Q4_K, 4) AH_ATTR(AH_GGML_Q4_K, 8) AH_ATTR(AH_GGML_Q4_K, 12)
    AH_ATTR(AH_GGML_Q6_K, 4) AH_ATTR(AH_GGML_Q6_K, 8) AH_ATTR(AH_GGML_Q6_K, 12)
#undef AH_ATTR
    for (uint32_t t : {AH_GGML_Q8_0, AH_GGML_Q5_0, AH_GGML_Q2_K, AH_GGML_Q3_K, AH_GGML_Q4_K, AH_GGML_Q6_K})
        for (int v = 0; v < 3; ++v)
            if (e == hipSuccess)
                e = hipFuncSetAttribute(stream_fn(t, v == 1, v == 2), hipFuncAttributeMaxDynamicSharedMemorySize, lim);
    for (int v = 0; v < 2; ++v)
        if (e == hipSuccess)
            e = hipFuncSetAttribute(stream_fn(kMixedType, v == 1), hipFuncAttributeMaxDynamicSharedMemorySize, lim);
    for (uint32_t t : {(uint32_t)kMixedType, (uint32_t)AH_GGML_Q8_0, (uint32_t)AH_GGML_Q4_K, (uint32_t)AH_GGML_Q6_K})
        if (e == hipSuccess) e = hipFuncSetAttribute(seq_fn(t), hipFuncAttributeMaxDynamicSharedMemorySize, lim);
    for (uint32_t t : {AH_GGML_Q8_0, AH_GGML_Q5_0, AH_GGML_Q2_K, AH_GGML_Q3_K, AH_GGML_Q4_K, AH_GGML_Q6_K})
        if (e == hipSuccess) e = hipFuncSetAttribute(ffn_fn(t), hipFuncAttributeMaxDynamicSharedMemorySize, lim);
    return e;
}

hipError_t ah_launch_gemv(uint32_t type, const GemvPart &single, const GemvPart *d_parts,
                          const uint32_t *d_wg_part, uint32_t grid, uint32_t kpad_max, uint32_t nc,
                          unsigned long long *status, hipStream_t stream) {
    const size_t lds = ah_gemv_lds_bytes(nc, kpad_max);
    switch (type) {
    case AH_GGML_Q8_0:
        launch_type<AH_GGML_Q8_0>(nc, dim3(grid), lds, stream, single, d_parts, d_wg_part, kpad_max, status);
        break;
    case AH_GGML_Q5_0:
        launch_type<AH_GGML_Q5_0>(nc, dim3(grid), lds, stream, single, d_parts, d_wg_part, kpad_max, status);
        break;
    case AH_GGML_Q2_K:
        launch_type<AH_GGML_Q2_K>(nc, dim3(grid), lds, stream, single, d_parts, d_wg_part, kpad_max, status);
        break;
    case AH_GGML_Q3_K:
        launch_type<AH_GGML_Q3_K>(nc, dim3(grid), lds, stream, single, d_parts, d_wg_part, kpad_max, status);
        break;
    case AH_GGML_Q4_K:
        launch_type<AH_GGML_Q4_K>(nc, dim3(grid), lds, stream, single, d_parts, d_wg_part, kpad_max, status);
        break;
    case AH_GGML_Q6_K:
        launch_type<AH_GGML_Q6_K>(nc, dim3(grid), lds, stream, single, d_parts, d_wg_part, kpad_max, status);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <uint32_t SRC>
static hipError_t launch_operand(const OperandArgs &o, hipStream_t stream) {
    const uint32_t nbp = o.kpad / 32;  // kpad <= AH_MAX_N_IN: <= 1024 blocks
    const dim3 grid(o.n_tok);
    if (nbp <= 64) hipLaunchKernelGGL((gemm_operand_kernel<SRC, 1, 256>), grid, dim3(256), 0, stream, o);
    else if (nbp <= 256) hipLaunchKernelGGL((gemm_operand_kernel<SRC, 1, 1024>), grid, dim3(1024), 0, stream, o);
    else if (nbp <= 512) hipLaunchKernelGGL((gemm_operand_kernel<SRC, 2, 1024>), grid, dim3(1024), 0, stream, o);
    else if (nbp <= 1024) hipLaunchKernelGGL((gemm_operand_kernel<SRC, 4, 1024>), grid, dim3(1024), 0, stream, o);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t ah_launch_gemm_operand(const OperandArgs &o, hipStream_t stream) {
    if (o.n_tok == 0) return hipSuccess;
    switch (o.src) {
    case AH_SRC_F32: return launch_operand<AH_SRC_F32>(o, stream);
    case AH_SRC_CODES: return launch_operand<AH_SRC_CODES>(o, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t ah_launch_quant(const QuantArgs &q, hipStream_t stream) {
    const size_t total = (size_t)q.n_tok * q.nb32;
    if (total == 0) return hipSuccess;
    size_t grid = (total + kThreads / 4 - 1) / (kThreads / 4);
    if (grid > 8192) grid = 8192;
    hipLaunchKernelGGL(quant_kernel, dim3((uint32_t)grid), dim3(kThreads), 0, stream, q);
    return hipGetLastError();
}

hipError_t ah_launch_swiglu_quant(const SwigluArgs &a, hipStream_t stream) {
    const uint64_t total = (uint64_t)a.n_tok * ((a.n_ff + 31) / 32);
    if (total == 0) return hipSuccess;
    uint64_t grid = (total + 7) / 8;  // 8 blocks per 256-thread workgroup
    if (grid > 8192) grid = 8192;
    hipLaunchKernelGGL(swiglu_quant_kernel, dim3((uint32_t)grid), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t ah_launch_scan(const uint8_t *w, uint64_t n_blocks, uint32_t block_bytes,
                          uint32_t off0, uint32_t off1, unsigned long long *d_bad, hipStream_t stream) {
    if (n_blocks == 0) return hipSuccess;
    uint64_t grid = (n_blocks + 255) / 256;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(scan_scales_kernel, dim3((uint32_t)grid), dim3(256), 0, stream, w, n_blocks,
                       block_bytes, off0, off1, d_bad);
    return hipGetLastError();
}
