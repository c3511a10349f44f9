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

namespace {

constexpr uint32_t kThreads = 256;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

AH_DEV u32x2 ah_ld64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0));
}

struct ActLds {
    int8_t *codes;   // [kpad]
    float *fsc;      // [kpad/32]   S_b * 2^-32
    int32_t *xs32;   // [kpad/32]   sum of codes per 32-block
    int32_t *xs16;   // [kpad/16]   sum of codes per 16-group
    float *red;      // [256 * NU]  unit partials of one tile
};

AH_DEV ActLds carve(uint8_t *smem, uint32_t kpad) {
    ActLds a;
    a.codes = reinterpret_cast<int8_t *>(smem);
    a.fsc = reinterpret_cast<float *>(smem + kpad);
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
};
AH_DEV QuadOut quant_quad(const void *x, uint32_t src, uint32_t n_in, size_t row_off, uint32_t b,
                          bool valid, unsigned long long *status, unsigned long long key_base) {
    const uint32_t q = threadIdx.x & 3;
    const uint32_t k0 = b * 32 + 8 * q;
    const uint32_t take = (valid && n_in > k0) ? (n_in - k0 < 8 ? n_in - k0 : 8) : 0;
    uint32_t bits[8];
    int64_t v64[8];
    uint32_t maxb = 0;
    uint64_t maxm = 0;
    if (src == AH_SRC_F32) {
        const uint32_t *xb = static_cast<const uint32_t *>(x) + row_off + k0;
        if (take == 8 && (reinterpret_cast<uintptr_t>(xb) & 15) == 0) {
            const u32x4 a = reinterpret_cast<const u32x4 *>(xb)[0], c = reinterpret_cast<const u32x4 *>(xb)[1];
            bits[0] = a.x; bits[1] = a.y; bits[2] = a.z; bits[3] = a.w;
            bits[4] = c.x; bits[5] = c.y; bits[6] = c.z; bits[7] = c.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) bits[i] = (uint32_t)i < take ? xb[i] : 0u;
        }
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
        const int64_t *xv = static_cast<const int64_t *>(x) + row_off + k0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            v64[i] = (uint32_t)i < take ? xv[i] : 0;
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
    QuadOut o;
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
                uint64_t m;
                bool n;
                if (src == AH_SRC_F32) {
                    (void)ah_to_q32_mag(bits[i], m, n);  // padded lanes are +0: code 0
                } else {
                    n = v64[i] < 0;
                    m = n ? 0ull - (uint64_t)v64[i] : (uint64_t)v64[i];
                }
                const int c = ah_act_code(m, n, e, bad);
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
    return o;
}

// Fill the LDS activation of part P: blocks past n_in (up to kpad) are zero, so ragged rows need
// no special case -- padded lanes contribute nothing to any dot or code sum.
AH_DEV void load_activation(const GemvPart &P, uint32_t kpad, const ActLds &A,
                            unsigned long long *status) {
    const uint32_t nb32 = (P.n_in + 31) / 32, nbp = kpad / 32, q = threadIdx.x & 3;
    for (uint32_t base = 0; base < nbp; base += kThreads / 4) {
        const uint32_t b = base + threadIdx.x / 4;
        const bool valid = b < nb32;
        QuadOut o;
        float fsc = 0.0f;
        if (P.src == AH_SRC_CODES) {
            const uint32_t k0 = b * 32 + 8 * q;
            const uint32_t take = (valid && P.n_in > k0) ? (P.n_in - k0 < 8 ? P.n_in - k0 : 8) : 0;
            const int8_t *c = static_cast<const int8_t *>(P.x) + k0;
            o.c0 = o.c1 = 0;
            int s8 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int v = (uint32_t)i < take ? (int)c[i] : 0;
                if (i < 4)
                    o.c0 |= (uint32_t)(v & 0xff) << (8 * i);
                else
                    o.c1 |= (uint32_t)(v & 0xff) << (8 * (i - 4));
                s8 += v;
            }
            o.s16 = s8 + (int)quad_xor1((uint32_t)s8);
            o.s32 = o.s16 + (int)quad_xor2((uint32_t)o.s16);
            if (valid) fsc = (float)P.scales[b] * 0x1p-32f;
        } else {
            o = quant_quad(P.x, P.src, P.n_in, 0, b, valid, status, 0);
            fsc = o.e < 0 ? 0.0f : __builtin_ldexpf(1.0f, o.e - 32);
        }
        if (b < nbp) {
            u32x2 *dst = reinterpret_cast<u32x2 *>(A.codes + 32 * b + 8 * q);
            *dst = (u32x2){o.c0, o.c1};
            if (q == 0) {
                A.fsc[b] = fsc;
                A.xs32[b] = o.s32;
                A.xs16[2 * b] = o.s16;
            } else if (q == 2) {
                A.xs16[2 * b + 1] = o.s16;
            }
        }
    }
}

// ---- per-family units: load (issued early) and compute ---------------------------------------

// Q8_0 block b (format/quant.rs:238-250): f16 d at byte 0, 32 int8 codes at 2..33; blocks are
// 2-byte aligned, so the 40-byte window from the 4-aligned address below is realigned.
struct UnitQ8 {
    u32x4 a0, a1;
    u32x2 a2;
    uint32_t sh;
};
AH_DEV void load_q8(__amdgpu_buffer_rsrc_t rs, uint32_t blk, UnitQ8 &u) {
    const uint32_t base = blk & ~3u;
    u.sh = blk & 3u;
    u.a0 = ah_ld128(rs, base);
    u.a1 = ah_ld128(rs, base + 16);
    u.a2 = ah_ld64(rs, base + 32);
}
AH_DEV float comp_q8(const UnitQ8 &u, uint32_t b, const ActLds &A, int32_t *dots) {
    const uint32_t w[10] = {u.a0.x, u.a0.y, u.a0.z, u.a0.w, u.a1.x, u.a1.y, u.a1.z, u.a1.w, u.a2.x, u.a2.y};
    const uint32_t d16 = (u.sh ? (w[0] >> 16) : w[0]) & 0xffffu;
    const u32x4 *xv = reinterpret_cast<const u32x4 *>(A.codes + 32 * b);
    const u32x4 x0 = xv[0], x1 = xv[1];
    const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    int32_t D = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t c = u.sh ? w[i + 1] : ah_alignbyte(w[i + 1], w[i], 2);
        D = ah_sdot4(c, xw[i], D);
    }
    if (dots) dots[b] = D;
    return ah_f16_bits_to_f32(d16) * A.fsc[b] * (float)D;
}

// get_scale_min_k4 (format/quant.rs:482-491) on the 12 packed bytes held in three dwords.
AH_DEV uint32_t sbyte(uint32_t s0, uint32_t s1, uint32_t s2, int i) {
    const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (w >> (8 * (i & 3))) & 0xffu;
}
template <int J>
AH_DEV void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &m) {
    if (J < 4) {
        sc = sbyte(s0, s1, s2, J) & 63;
        m = sbyte(s0, s1, s2, J + 4) & 63;
    } else {
        sc = (sbyte(s0, s1, s2, J + 4) & 0xF) | ((sbyte(s0, s1, s2, J - 4) >> 6) << 4);
        m = (sbyte(s0, s1, s2, J + 4) >> 4) | ((sbyte(s0, s1, s2, J) >> 6) << 4);
    }
}

// Q4_K super-block s (format/quant.rs:481-510): d, dmin, 12 packed 6-bit (scale, min) pairs,
// 128 bytes of nibbles; sub-block j takes the low (j even) / high (j odd) nibbles of
// qs[32*(j/2) + l].  Only the qs windows a ragged row uses are loaded.
struct UnitQ4 {
    u32x4 v[9];
};
AH_DEV void load_q4(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t npairs, UnitQ4 &u) {
    u.v[0] = ah_ld128(rs, off);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        if ((uint32_t)p < npairs) {
            u.v[1 + 2 * p] = ah_ld128(rs, off + 16 + 32 * p);
            u.v[2 + 2 * p] = ah_ld128(rs, off + 32 + 32 * p);
        } else {
            u.v[1 + 2 * p] = (u32x4){0u, 0u, 0u, 0u};
            u.v[2 + 2 * p] = (u32x4){0u, 0u, 0u, 0u};
        }
    }
}
template <int P>
AH_DEV float q4k_pair(const UnitQ4 &u, float fd, float fdm, uint32_t g0, uint32_t nb32,
                      const ActLds &A, int32_t *dots) {
    const uint32_t q[8] = {u.v[1 + 2 * P].x, u.v[1 + 2 * P].y, u.v[1 + 2 * P].z, u.v[1 + 2 * P].w,
                           u.v[2 + 2 * P].x, u.v[2 + 2 * P].y, u.v[2 + 2 * P].z, u.v[2 + 2 * P].w};
    const u32x4 *xv = reinterpret_cast<const u32x4 *>(A.codes + 32 * g0);
    const u32x4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
    const uint32_t xl[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const uint32_t xh[8] = {x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
    int32_t Dlo = 0, Dhi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        Dlo = ah_sdot4(q[i] & 0x0F0F0F0Fu, xl[i], Dlo);
        Dhi = ah_sdot4((q[i] >> 4) & 0x0F0F0F0Fu, xh[i], Dhi);
    }
    int sl, ml, shh, mh;
    q4k_scale_min<2 * P>(u.v[0].y, u.v[0].z, u.v[0].w, sl, ml);
    q4k_scale_min<2 * P + 1>(u.v[0].y, u.v[0].z, u.v[0].w, shh, mh);
    if (dots) {
        dots[g0] = Dlo;
        if (g0 + 1 < nb32) dots[g0 + 1] = Dhi;  // a ragged row ends on an odd sub-block
    }
    const float tlo = fd * (float)(sl * Dlo) - fdm * (float)(ml * A.xs32[g0]);
    const float thi = fd * (float)(shh * Dhi) - fdm * (float)(mh * A.xs32[g0 + 1]);
    return A.fsc[g0] * tlo + A.fsc[g0 + 1] * thi;
}
AH_DEV float comp_q4(const UnitQ4 &u, uint32_t s, uint32_t npairs, uint32_t nb32, const ActLds &A,
                     int32_t *dots) {
    const float fd = ah_f16_bits_to_f32(u.v[0].x & 0xffffu), fdm = ah_f16_bits_to_f32(u.v[0].x >> 16);
    const uint32_t g = 8 * s;
    float acc = q4k_pair<0>(u, fd, fdm, g, nb32, A, dots);
    if (npairs > 1) acc += q4k_pair<1>(u, fd, fdm, g + 2, nb32, A, dots);
    if (npairs > 2) acc += q4k_pair<2>(u, fd, fdm, g + 4, nb32, A, dots);
    if (npairs > 3) acc += q4k_pair<3>(u, fd, fdm, g + 6, nb32, A, dots);
    return acc;
}

// Q6_K super-block s (format/quant.rs:556-599): ql[128] @0, qh[64] @128, int8 sc[16] @192,
// f16 d @208.  Element 128n + 32t + l = (nibble t/2 of ql[64n + 32(t&1) + l]
// | ((qh[32n + l] >> 2t) & 3) << 4) - 32.  Super-blocks are 2-byte aligned: the 216-byte window
// from the 4-aligned address below is realigned in registers.
struct UnitQ6 {
    u32x4 v[13];
    u32x2 t;
    uint32_t sh;
};
AH_DEV void load_q6(__amdgpu_buffer_rsrc_t rs, uint32_t addr, UnitQ6 &u) {
    const uint32_t base = addr & ~3u;
    u.sh = addr & 3u;
#pragma unroll
    for (int i = 0; i < 13; ++i) u.v[i] = ah_ld128(rs, base + 16 * i);
    u.t = ah_ld64(rs, base + 208);
}
AH_DEV float comp_q6(const UnitQ6 &u, uint32_t s, uint32_t nb32, uint32_t nb16, const ActLds &A,
                     int32_t *dots16) {
    uint32_t w[54];
#pragma unroll
    for (int i = 0; i < 13; ++i) {
        w[4 * i] = u.v[i].x;
        w[4 * i + 1] = u.v[i].y;
        w[4 * i + 2] = u.v[i].z;
        w[4 * i + 3] = u.v[i].w;
    }
    w[52] = u.t.x;
    w[53] = u.t.y;
    const uint32_t sh = u.sh;
    auto V = [&](int i) -> uint32_t { return ah_alignbyte(w[i + 1], w[i], sh); };
    const float fd = ah_f16_bits_to_f32(V(52) & 0xffffu);
    float acc = 0.0f;
#pragma unroll
    for (int n = 0; n < 2; ++n) {
        uint32_t qh[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) qh[i] = V(32 + 8 * n + i);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t g = 8 * s + 4 * n + t;
            if (g >= nb32) break;
            const u32x4 *xv = reinterpret_cast<const u32x4 *>(A.codes + 32 * g);
            const u32x4 x0 = xv[0], x1 = xv[1];
            const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            int32_t Dlo = 0, Dhi = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t qlw = V(16 * n + 8 * (t & 1) + i);
                const uint32_t lo4 = t < 2 ? (qlw & 0x0F0F0F0Fu) : ((qlw >> 4) & 0x0F0F0F0Fu);
                const uint32_t uu = lo4 | (((qh[i] >> (2 * t)) & 0x03030303u) << 4);
                if (i < 4)
                    Dlo = ah_sdot4(uu, xw[i], Dlo);
                else
                    Dhi = ah_sdot4(uu, xw[i], Dhi);
            }
            Dlo -= 32 * A.xs16[2 * g];
            Dhi -= 32 * A.xs16[2 * g + 1];
            const uint32_t scw = V(48 + 2 * n + (t >> 1));
            const int sclo = (int)(int8_t)((scw >> (16 * (t & 1))) & 0xffu);
            const int schi = (int)(int8_t)((scw >> (16 * (t & 1) + 8)) & 0xffu);
            if (dots16) {
                dots16[2 * g] = Dlo;
                if (2 * g + 1 < nb16) dots16[2 * g + 1] = Dhi;  // ragged row ends on a 16-group
            }
            acc += A.fsc[g] * fd * (float)(sclo * Dlo + schi * Dhi);
        }
    }
    return acc;
}

template <int TYPE>
struct UnitOf;
template <>
struct UnitOf<AH_GGML_Q8_0> {
    typedef UnitQ8 T;
};
template <>
struct UnitOf<AH_GGML_Q4_K> {
    typedef UnitQ4 T;
};
template <>
struct UnitOf<AH_GGML_Q6_K> {
    typedef UnitQ6 T;
};

template <int TYPE>
AH_DEV void load_unit(__amdgpu_buffer_rsrc_t rs, const GemvPart &P, uint32_t row, uint32_t u,
                      typename UnitOf<TYPE>::T &x) {
    if constexpr (TYPE == AH_GGML_Q8_0) {
        load_q8(rs, row * P.row_bytes + 34 * u, x);
    } else if constexpr (TYPE == AH_GGML_Q4_K) {
        const uint32_t rem = P.n_in - 256 * u;
        load_q4(rs, row * P.row_bytes + 144 * u, rem >= 256 ? 4u : (rem + 63) / 64, x);
    } else {
        load_q6(rs, row * P.row_bytes + 210 * u, x);
    }
}

template <int TYPE>
AH_DEV float comp_unit(const GemvPart &P, uint32_t row, uint32_t u, const typename UnitOf<TYPE>::T &x,
                       const ActLds &A) {
    const uint32_t nb32 = (P.n_in + 31) / 32;
    if constexpr (TYPE == AH_GGML_Q8_0) {
        return comp_q8(x, u, A, P.dots ? P.dots + (size_t)row * nb32 : nullptr);
    } else if constexpr (TYPE == AH_GGML_Q4_K) {
        const uint32_t rem = P.n_in - 256 * u;
        return comp_q4(x, u, rem >= 256 ? 4u : (rem + 63) / 64, nb32, A,
                       P.dots ? P.dots + (size_t)row * nb32 : nullptr);
    } else {
        const uint32_t nb16 = (P.n_in + 15) / 16;
        return comp_q6(x, u, nb32, nb16, A, P.dots ? P.dots + (size_t)row * nb16 : nullptr);
    }
}

template <int TYPE, int NU>
__global__ void __launch_bounds__(kThreads)
    gemv_kernel(GemvPart single, const GemvPart *__restrict__ parts, uint32_t n_parts,
                uint32_t kpad_max, unsigned long long *status) {
    extern __shared__ __align__(16) uint8_t smem[];
    typedef typename UnitOf<TYPE>::T Unit;
    GemvPart P = single;
    if (parts) {
        uint32_t lo = 0, hi = n_parts;  // last part with wg_begin <= blockIdx.x
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) / 2;
            if (parts[mid].wg_begin <= blockIdx.x) lo = mid;
            else hi = mid;
        }
        P = parts[lo];
    }
    const uint32_t wg_local = blockIdx.x - P.wg_begin;
    const uint32_t kpad = (P.n_in + 255) / 256 * 256;
    const ActLds A = carve(smem, kpad_max);
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(P.w, (uint32_t)P.w_bytes);
    const uint32_t U = P.units, R = P.rows_per_tile, TU = R * U;
    const uint32_t n_tiles = (P.n_out + R - 1) / R;

    // (row, unit) of this thread's j-th unit in tile `tile`, or row = n_out when idle
    auto slot = [&](uint32_t tile, int j, uint32_t &row, uint32_t &u) {
        const uint32_t f = threadIdx.x + kThreads * j;
        row = P.n_out;
        u = 0;
        if (f < TU) {
            const uint32_t r = f / U;
            u = f - r * U;
            row = tile * R + r;
            if (row > P.n_out) row = P.n_out;
        }
    };

    Unit cur[NU], nxt[NU];
    uint32_t tile = wg_local;
    if (tile < n_tiles) {
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            uint32_t row, u;
            slot(tile, j, row, u);
            if (row < P.n_out) load_unit<TYPE>(rs, P, row, u, cur[j]);
        }
    }
    load_activation(P, kpad, A, status);
    __syncthreads();

    for (; tile < n_tiles; tile += P.wg_count) {
        const uint32_t next = tile + P.wg_count;
        if (next < n_tiles) {
#pragma unroll
            for (int j = 0; j < NU; ++j) {
                uint32_t row, u;
                slot(next, j, row, u);
                if (row < P.n_out) load_unit<TYPE>(rs, P, row, u, nxt[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            uint32_t row, u;
            slot(tile, j, row, u);
            if (row < P.n_out) A.red[threadIdx.x + kThreads * j] = comp_unit<TYPE>(P, row, u, cur[j], A);
        }
        __syncthreads();
        // row sums in fixed order: G lanes per row, G a power of two with R*G <= 256
        uint32_t G = 64;
        while (G > 1 && R * G > kThreads) G >>= 1;
        const uint32_t r = threadIdx.x / G, gl = threadIdx.x & (G - 1);
        float s = 0.0f;
        if (r < R)
            for (uint32_t i = gl; i < U; i += G) s += A.red[r * U + i];
        for (uint32_t o = 1; o < G; o <<= 1) s += __shfl_xor(s, (int)o, 64);
        const uint32_t row = tile * R + r;
        if (r < R && gl == 0 && row < P.n_out) P.y[row] = s;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NU; ++j) cur[j] = nxt[j];
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

// Device-side f16 scale scan of a payload: flags any Inf/NaN d / dmin word.
__global__ void scan_scales_kernel(const uint8_t *w, uint64_t n_blocks, uint32_t block_bytes,
                                   uint32_t off0, uint32_t off1, int *bad) {
    for (uint64_t b = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; b < n_blocks;
         b += (uint64_t)gridDim.x * blockDim.x) {
        const uint8_t *p = w + b * block_bytes;
        uint32_t h0 = p[off0] | (p[off0 + 1] << 8);
        bool nf = ((h0 >> 10) & 0x1f) == 0x1f;
        if (off1 != off0) {
            uint32_t h1 = p[off1] | (p[off1 + 1] << 8);
            nf |= ((h1 >> 10) & 0x1f) == 0x1f;
        }
        if (nf) atomicOr(bad, 1);
    }
}

}  // namespace

// ---- launchers (called from ah_abi.cpp) ----

// Units per thread per tile for each family (register budget of the double-buffered unit).
uint32_t ah_gemv_nu(uint32_t type) { return type == AH_GGML_Q8_0 ? 4u : 1u; }

size_t ah_gemv_lds_bytes(uint32_t type, uint32_t kpad_max) {
    return kpad_max + (size_t)kpad_max / 32 * 8 + (size_t)kpad_max / 16 * 4 +
           (size_t)kThreads * ah_gemv_nu(type) * 4;
}

hipError_t ah_launch_gemv(uint32_t type, const GemvPart &single, const GemvPart *d_parts,
                          uint32_t n_parts, uint32_t grid, uint32_t kpad_max,
                          unsigned long long *status, hipStream_t stream) {
    const size_t lds = ah_gemv_lds_bytes(type, kpad_max);
    switch (type) {
    case AH_GGML_Q8_0:
        hipLaunchKernelGGL((gemv_kernel<AH_GGML_Q8_0, 4>), dim3(grid), dim3(kThreads), lds, stream,
                           single, d_parts, n_parts, kpad_max, status);
        break;
    case AH_GGML_Q4_K:
        hipLaunchKernelGGL((gemv_kernel<AH_GGML_Q4_K, 1>), dim3(grid), dim3(kThreads), lds, stream,
                           single, d_parts, n_parts, kpad_max, status);
        break;
    case AH_GGML_Q6_K:
        hipLaunchKernelGGL((gemv_kernel<AH_GGML_Q6_K, 1>), dim3(grid), dim3(kThreads), lds, stream,
                           single, d_parts, n_parts, kpad_max, status);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t ah_launch_quant(const QuantArgs &q, hipStream_t stream) {
    const size_t total = (size_t)q.n_tok * q.nb32;
    if (total == 0) return hipSuccess;
    size_t grid = (total + kThreads / 4 - 1) / (kThreads / 4);
    if (grid > 8192) grid = 8192;
    hipLaunchKernelGGL(quant_kernel, dim3((uint32_t)grid), dim3(kThreads), 0, stream, q);
    return hipGetLastError();
}

hipError_t ah_launch_scan(const uint8_t *w, uint64_t n_blocks, uint32_t block_bytes,
                          uint32_t off0, uint32_t off1, int *d_bad, hipStream_t stream) {
    if (n_blocks == 0) return hipSuccess;
    uint64_t grid = (n_blocks + 255) / 256;
    if (grid > 4096) grid = 4096;
    hipLaunchKernelGGL(scan_scales_kernel, dim3((uint32_t)grid), dim3(256), 0, stream, w, n_blocks,
                       block_bytes, off0, off1, d_bad);
    return hipGetLastError();
}
