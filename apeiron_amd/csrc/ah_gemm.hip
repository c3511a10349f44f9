// ah_gemm.hip -- prefill GEMM (N > 1) over GGUF Q8_0 / Q4_K / Q6_K payloads on gfx950 MFMA.
//
// Reference semantics: column c of matmat_q8act (kern/matmat.rs:134) is matvec_q8act on token c;
// the reference's GEMMs (kern/gemm.rs:488-580 Q8_0, chart/kcols.rs:1399-1518 Q4_K / Q6_K) fold
// sum_b d_rb * S_cb * D_rcb with exact integer group dots D.
//
// MI355X design (the f16 design; an int8-MFMA design for Q8_0 follows gemm_rb_kernel).  After an
// int8 MFMA every 32-block needs an f32 fold per output element (convert, scale, accumulate).
// Instead both operands are fed to v_mfma_f32_32x32x16_f16 as exact small integers:
//   * the activation operand is xq * 2^(e_b - E_tok) in f16 (the quantizer's power-of-two block
//     scale S_b = 2^e_b folded in exactly; E_tok is the token's largest block exponent, applied
//     once at the end), so the MFMA itself applies the activation scale;
//   * the weight operand is the integer code (Q8_0 q, Q6_K u-32) or, for Q4_K, sc_j * q (<= 945),
//     exact in f16.
// Every product is exact.  For Q8_0 a block's partial sums stay below 2^24 units of its smallest
// term (|q * xq| <= 127 * 127, 32 terms), so a Q8_0 block result is exactly 2^(e_b-E) * D_b.  The
// K-quants accumulate a whole super-block (Q6_K) or its sc-weighted sub-blocks (Q4_K) in one MFMA
// accumulator, whose sums pass 2^24 (up to ~1.2e5 per Q4_K product, ~5.2e5 per Q6_K element) and
// round: each accumulation step rounds at 2^-24 relative, so a super-block's sum is off by at most
// ~256 * 2^-24 ~= 1.5e-5 of the sum of its terms' magnitudes, inside the contract's 1e-4 *
// sum|w * xhat| tolerance.  What remains per output element is one FMA per weight-scale change:
// per 32-block (Q8_0 d), per 256-super-block (Q6_K d; Q4_K d, plus one FMA for the dmin*m*X term,
// which rides on one extra MFMA per super-block).
//
// Tiling (gemm_rb_kernel below): a workgroup is 4 (or 2) waves; wave w owns 32 weight rows (the
// MFMA N/column dimension, so the weight scale is one value per lane) and the workgroup's 128
// tokens (64 for Q4_K) as 32-token MFMA row tiles.  The f16 activation slice of each 64-deep K
// stage goes global -> LDS into a ring of 4 (or 2) slots shared by the waves; each wave reads its
// own weight rows straight from the GGUF bytes ahead of use and converts them in registers.  One
// launch may cover several projections of one input (parts).  Split-K writes partials that one
// pass per grouped call reduces in fixed order.
#include "ah_internal.h"
#include "ah_swiglu.h"
#include "ah_units.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;
constexpr int kKS = 64;                // K depth of one LDS stage


AH_DEV f32x16 mfma(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

AH_DEV f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
AH_DEV uint32_t as_u(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// 4 signed int8 codes -> 4 exact f16 (two f16x2 words): f16 bits 0x6400|(c^0x80) = 1024 + c + 128.
AH_DEV void i8x4_to_f16(uint32_t c, uint32_t &lo, uint32_t &hi) {
    const uint32_t u = c ^ 0x80808080u;
    const f16x2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
    hi = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}

// 4 unsigned 5-bit values (bytes) -> 4 exact f16 of (u - 16).
AH_DEV void u5x4_to_f16(uint32_t u, uint32_t &lo, uint32_t &hi) {
    const f16x2 bias = {(_Float16)1040.0f, (_Float16)1040.0f};
    lo = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
    hi = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}

// 4 unsigned 6-bit values (bytes) -> 4 exact f16 of (u - 32).
AH_DEV void u6x4_to_f16(uint32_t u, uint32_t &lo, uint32_t &hi) {
    const f16x2 bias = {(_Float16)1056.0f, (_Float16)1056.0f};
    lo = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
    hi = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}

// 4 bytes b (the nibble q as q or 16 q) -> 4 f16 (1024 + b) * sc2 + off2 (exact sc*q for the
// scale pairs the Q4_K stage passes).
AH_DEV void nib4_times(uint32_t n, f16x2 sc2, f16x2 off2, uint32_t &lo, uint32_t &hi) {
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, n, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, n, 0x04030402u);
    lo = as_u(__builtin_elementwise_fma(as_h2(a), sc2, off2));
    hi = as_u(__builtin_elementwise_fma(as_h2(b), sc2, off2));
}

AH_DEV f16x8 pack8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const u32x4 v = {a, b, c, d};
    return __builtin_bit_cast(f16x8, v);
}

// A part of the launch: logical workgroups [wg_begin, next part's wg_begin) are its tiles x splits.
struct GemmPartArgs {
    const uint8_t *w;
    float *y;                  // [n_tok][n_out] (splits == 1) or partials [splits][n_tok][n_out]
    uint32_t w_bytes, row_bytes, n_out;
    uint32_t stages_per_split; // K stages of 64 per split (multiple of the kernel's unroll)
    uint32_t splits, wg_begin;
    uint32_t tok_tiles;        // token tiles of the part's type
    uint32_t type;             // GGUF type (read by the mixed K-quant kernel)
    uint64_t key0;             // added to the part's output refusal keys (GemmPartDesc::key0)
};
struct GemmArgs {
    GemmPartArgs p[kGemmMaxParts];
    uint32_t n_parts, n_in, n_tok, kpad;
    const _Float16 *xh;        // [n_tok][kpad]
    const _Float16 *xf;        // the same in fragment order (OperandArgs::xf), for the tile design
    const _Float16 *xmin;      // Q4_K: [n_tok][kpad/256][16] split code sums (see quant pass)
    const _Float16 *xmin16;    // Q2_K / Q3_K tiles: [n_tok][kpad/256][16] 16-group code sums
    const float *tok_scale;    // [n_tok]; bit 0 set: the token is served by the exact path
    unsigned long long *status;
    const int8_t *fcodes;      // [n_tok][n_in] codes of flagged tokens
    const int64_t *fscales;    // [n_tok][nb32] their scales
    const int8_t *xc;          // int8 design: codes [n_tok][kpad] (zero past n_in)
    const uint32_t *xsp;       // int8 design: [n_tok][kpad/32] block factors 2^(e_b - E_tok), bf16 x2
    const uint32_t *xsx;       // int8 Q4_K: [n_tok][kpad/32] 2^(e_b - E_tok) X_b as bf16 (hi, lo)
    uint32_t n_wg;             // real workgroup count over all parts
    GemmFfn ffn;               // kFormTileFfn: the up projection and the hidden QuantAct outputs
};

constexpr uint32_t kOob = 0xFFFFFFF0u;  // a buffer offset past any operand: reads zeros

// ---- register-blocked kernel ----------------------------------------------------------------
//
// A workgroup is 4 waves.  Wave w owns NN 32-row MFMA column tiles (n) of weight rows and all NM
// 32-token row tiles (m) of the workgroup's tokens, so every activation fragment read from LDS
// feeds NN MFMAs and every dequantized weight fragment feeds NM.  The VALU work per MFMA (weight
// dequantization over NM, plus the scale folds) is what bounds this kernel, so NM = 4 by default;
// LDS sustains the resulting 1 KB of fragment reads per MFMA.  The loop body is U stages of 64
// (Q8_0: U = 2, K-quants: U = 4 = one super-block), so the LDS buffer, the weight register set and the
// super-block position of each stage are compile-time: no runtime register indexing, no copies
// between register sets.
namespace rb {
constexpr int kNN = 1;                          // column tiles per wave
// A workgroup is W waves (each owns 32 weight rows) with an R-slot LDS ring; the host picks the
// form per GEMM shape (ah_gemm_pick_waves).
template <int W> constexpr int rows() { return W * 32 * kNN; }  // rows per workgroup
// Row (token) tiles per wave.  Q8_0 (a fold per block) and Q6_K (two operands per weight, see
// the Q6_K stage) are bound by VALU work per MFMA, so each dequantized weight fragment feeds 4
// token tiles.  Q4_K's dequantization is cheap and it is bound by the stalls of a single wave per
// SIMD instead: 2 token tiles halve the registers and the tile, so two of its workgroups share a
// CU at prefill sizes.  (Measured each way round: the other choice is 7-11% slower per type.)
template <int TYPE> constexpr int nm() { return TYPE == AH_GGML_Q4_K ? 2 : 4; }
// Parts one launch may hold (see the part lookup in the kernel).
template <int TYPE> constexpr uint32_t max_parts() { return ah_blk32(TYPE) ? 1u : kGemmMaxParts; }
uint32_t max_parts_of(uint32_t type) { return ah_blk32((int)type) ? 1u : kGemmMaxParts; }
template <int TYPE> constexpr int tok() { return 32 * nm<TYPE>(); }              // tokens per workgroup
template <int TYPE> constexpr int act_bytes() { return tok<TYPE>() * kKS * 2; }   // f16 slice of a stage
template <int TYPE> constexpr int buf_bytes() { return act_bytes<TYPE>(); }         // one ring slot
// Q4_K split code sums of a super-block (32 bytes per token), loaded once per super-block by one
// 16-byte direct-to-LDS instruction per wave into a region of their own after the ring: wave w's
// lanes l < xlanes<W>() take tokens [w * xtok<W>(), +xtok<W>()), two lanes per token; its other
// lanes read out of range into the rest of the wave's 1 KB.
template <int W> constexpr int xtok() { return tok<AH_GGML_Q4_K>() / W; }
template <int W> constexpr int xlanes() { return 2 * xtok<W>(); }
template <int TYPE, int W> constexpr int xregion() { return TYPE == AH_GGML_Q4_K ? W * 1024 : 0; }
template <int TYPE, int W, int R> constexpr int lds_bytes() { return R * buf_bytes<TYPE>() + xregion<TYPE, W>(); }
// Split granularity in stages (Q8_0 pairs, K-quant super-blocks); the loop body is 4 stages.
template <int TYPE> constexpr int unroll() { return ah_blk32(TYPE) ? 2 : 4; }
// Weight register sets and how many stages ahead they are fetched (Q6_K's 27-register set
// allows only two sets within the 256-register budget).
// The prologue replays ring - 1 notional stages, so a fetch is at most ring - 1 stages ahead.
template <int TYPE, int R> constexpr int dw() { return TYPE == AH_GGML_Q6_K || R < 3 ? 1 : 2; }
template <int TYPE, int R> constexpr int nw() { return dw<TYPE, R>() == 1 ? 2 : 4; }
// Per-wave direct-to-LDS instructions of one stage's slice (16-byte loads, 1 KB per
// instruction), and of a super-block's Q4_K split sums (issued at its first stage).
template <int TYPE, int W> constexpr int an() { return tok<TYPE>() * kKS * 2 / 1024 / W; }
template <int TYPE> constexpr int xn() { return TYPE == AH_GGML_Q4_K ? 1 : 0; }
// The vmcnt the top of stage u (of a super-block) waits for.  The stage's slice was issued R - 1
// stages earlier (R ring slots); after it came the slices of the R - 2 stages that follow, the
// split sums issued at a super-block's first stage (before that stage's slice, R = 4) and the
// weight fetches.  Only the slices and split sums are counted: the compiler merges or drops
// weight loads that coincide across the unrolled stages (the Q6_K d dword is one address for a
// whole super-block), so their number per stage is not fixed, while every slice instruction is
// issued.  Vector memory loads complete in issue order, so vmcnt <= the slice instructions issued
// since makes the stage's slice (and any load older than it, such as the split sums issued just
// before the slice of a super-block's last stage) complete, whatever the weight loads' count.
template <int TYPE, int W, int R> constexpr int wait_count(int u) {
    int n = 0;
    for (int v = u - (R - 2); v < u; ++v) n += an<TYPE, W>() + (((v % 4) + 4) % 4 == 0 ? xn<TYPE>() : 0);
    return n;
}
inline uint32_t tok_of(uint32_t type) {
    return type == AH_GGML_Q4_K ? tok<AH_GGML_Q4_K>() : type == AH_GGML_Q6_K ? tok<AH_GGML_Q6_K>() : tok<AH_GGML_Q8_0>();
}

}  // namespace rb

// Weight bytes of one stage for the lane's NN rows, fetched a stage ahead.  Ordinary (not
// non-temporal) loads: the workgroups of the other token tiles read the same bytes from L2.
//   Q8_0: per row n and block bb, v[2n+bb] = the 16 codes of the lane half (4-aligned window),
//         s[4n+2bb] = the dword after the window, s[4n+2bb+1] = the dword holding d.
//   Q4_K: v[2n] = super-block header (read at the super-block's first stage only),
//         v[2n+1] = the lane half's 16 bytes of qs chunk P.
//   Q6_K (one row per lane): stage P of a super-block covers half n = P/2, low (P even) or high
//         nibbles: v[0..3] = 64 bytes from ql[64n + 8h], v[4..5] = 32 bytes from qh[32n + 8h],
//         s[0..1] = 8 bytes from sc[4P], s[2] = the dword holding d (all from 4-aligned
//         addresses below, realigned by the super-block's offset mod 4).
struct WRb {
    u32x4 v[6];
    uint32_t s[8];
};

template <int TYPE, int P, int NN>
AH_DEV WRb fetch_rb(__amdgpu_buffer_rsrc_t rs, const uint32_t (&rb)[NN], const bool (&rl)[NN],
                    uint32_t st, uint32_t n_in, int h, bool live) {
    WRb w;
#pragma unroll
    for (int i = 0; i < 6; ++i) w.v[i] = (u32x4){0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) w.s[i] = 0u;
    const uint32_t k0 = st * kKS;
    if constexpr (TYPE == AH_GGML_Q8_0) {
        const uint32_t b = k0 / 32;
        const bool l0 = live && b * 32 < n_in, l1 = live && (b + 1) * 32 < n_in;
#pragma unroll
        for (int n = 0; n < NN; ++n) {
            const uint32_t blk0 = rb[n] + 34 * b, blk1 = blk0 + 34;
            const bool m0 = l0 && rl[n], m1 = l1 && rl[n];
            const uint32_t c0 = (blk0 + 2 + 16 * h) & ~3u, c1 = (blk1 + 2 + 16 * h) & ~3u;
            w.v[2 * n] = ah_ld128(rs, m0 ? c0 : kOob);
            w.s[4 * n] = ah_ld32(rs, m0 ? c0 + 16 : kOob);
            w.s[4 * n + 1] = ah_ld32(rs, m0 ? (blk0 & ~3u) : kOob);
            w.v[2 * n + 1] = ah_ld128(rs, m1 ? c1 : kOob);
            w.s[4 * n + 2] = ah_ld32(rs, m1 ? c1 + 16 : kOob);
            w.s[4 * n + 3] = ah_ld32(rs, m1 ? (blk1 & ~3u) : kOob);
        }
    } else if constexpr (TYPE == AH_GGML_Q5_0) {
        // per block the 6 dwords from its 4-aligned start: d, qh and all 16 qs bytes (both lane
        // halves need every qs byte: half 0 the low nibbles, half 1 the high ones)
        const uint32_t b = k0 / 32;
        const bool l0 = live && b * 32 < n_in, l1 = live && (b + 1) * 32 < n_in;
#pragma unroll
        for (int n = 0; n < NN; ++n) {
            const uint32_t c0 = (rb[n] + 22 * b) & ~3u, c1 = (rb[n] + 22 * (b + 1)) & ~3u;
            const bool m0 = l0 && rl[n], m1 = l1 && rl[n];
            w.v[2 * n] = ah_ld128(rs, m0 ? c0 : kOob);
            w.s[4 * n] = ah_ld32(rs, m0 ? c0 + 16 : kOob);
            w.s[4 * n + 1] = ah_ld32(rs, m0 ? c0 + 20 : kOob);
            w.v[2 * n + 1] = ah_ld128(rs, m1 ? c1 : kOob);
            w.s[4 * n + 2] = ah_ld32(rs, m1 ? c1 + 16 : kOob);
            w.s[4 * n + 3] = ah_ld32(rs, m1 ? c1 + 20 : kOob);
        }
    } else if constexpr (TYPE == AH_GGML_Q6_K) {
        static_assert(NN == 1, "Q6_K stages one row per lane");
        const uint32_t sb = rb[0] + 210 * (k0 / 256), nh = P / 2;
        const bool m = live && rl[0];
        const uint32_t aql = (sb + 64 * nh + 8 * h) & ~3u, aqh = (sb + 128 + 32 * nh + 8 * h) & ~3u;
#pragma unroll
        for (int i = 0; i < 4; ++i) w.v[i] = ah_ld128(rs, m ? aql + 16 * i : kOob);
        w.v[4] = ah_ld128(rs, m ? aqh : kOob);
        w.v[5] = ah_ld128(rs, m ? aqh + 16 : kOob);
        const uint32_t asc = (sb + 192 + 4 * P) & ~3u;
        w.s[0] = ah_ld32(rs, m ? asc : kOob);
        w.s[1] = ah_ld32(rs, m ? asc + 4 : kOob);
        w.s[2] = ah_ld32(rs, m ? (sb + 208) & ~3u : kOob);
    } else {
#pragma unroll
        for (int n = 0; n < NN; ++n) {
            const uint32_t sb = rb[n] + 144 * (k0 / 256);
            const bool m = live && rl[n];
            if constexpr (P == 0) w.v[2 * n] = ah_ld128(rs, m ? sb : kOob);
            else w.v[2 * n] = (u32x4){0u, 0u, 0u, 0u};
            w.v[2 * n + 1] = ah_ld128(rs, m ? sb + 16 + 32 * P + 16 * h : kOob);
        }
    }
    return w;
}

// Q4_K 6-bit scale (MIN = false) or min (MIN = true) of sub-block J from the 12 packed bytes
// (get_scale_min_k4, format/quant.rs:200-213).
template <int J, bool MIN>
AH_DEV uint32_t q4k_scale(uint32_t s0, uint32_t s1, uint32_t s2) {
    auto byte = [&](int i) -> uint32_t {
        const uint32_t wv = i < 4 ? s0 : (i < 8 ? s1 : s2);
        return (wv >> (8 * (i & 3))) & 0xffu;
    };
    if constexpr (J < 4) return byte(J + (MIN ? 4 : 0)) & 63;
    else if constexpr (!MIN) return (byte(J + 4) & 0xF) | ((byte(J - 4) >> 6) << 4);
    else return (byte(J + 4) >> 4) | ((byte(J) >> 6) << 4);
}

// ---- exact path for tokens the f16 operand cannot carry ----------------------------------------
//
// A token flagged by the operand pass (a nonzero block more than kF16Band binades below its largest)
// is recomputed per row from its codes and power-of-two scales, like the GEMV: exact integer group
// dots, folded in f32 with the block scale S_b * 2^-32 (an exact f32 power of two for every S_b a
// QuantAct can hold).  Units are Q8_0 blocks / K-quant super-blocks in [u_lo, u_hi), every second
// one from `first`.  Byte loads throughout: this path serves rare, pathological activations.
AH_DEV float s_of(const int64_t *sc, uint32_t b) { return (float)sc[b] * 0x1p-32f; }  // exact for 2^e
AH_DEV uint32_t byte_at(const uint8_t *p, uint32_t i) { return p[i]; }
AH_DEV float f16_at(const uint8_t *p) { return ah_f16_bits_to_f32(byte_at(p, 0) | (byte_at(p, 1) << 8)); }

template <int TYPE>
AH_DEV float exact_row(const uint8_t *row, const int8_t *xq, const int64_t *sc, uint32_t n_in,
                       uint32_t u_lo, uint32_t u_hi, uint32_t first) {
    float acc = 0.0f;
    for (uint32_t u = u_lo + first; u < u_hi; u += 2) {
        if constexpr (TYPE == AH_GGML_Q8_0) {
            const uint8_t *blk = row + 34 * u;
            int D = 0;
            for (uint32_t l = 0; l < 32 && 32 * u + l < n_in; ++l)
                D += (int)(int8_t)byte_at(blk, 2 + l) * (int)xq[32 * u + l];
            acc += s_of(sc, u) * (f16_at(blk) * (float)D);
        } else if constexpr (TYPE == AH_GGML_Q5_0) {  // format/quant.rs:263-297
            const uint8_t *blk = row + 22 * u;
            const uint32_t qh = byte_at(blk, 2) | (byte_at(blk, 3) << 8) | (byte_at(blk, 4) << 16) | (byte_at(blk, 5) << 24);
            int D = 0;
            for (uint32_t l = 0; l < 32 && 32 * u + l < n_in; ++l) {
                const uint32_t j = l & 15u, nib = (byte_at(blk, 6 + j) >> (l < 16 ? 0 : 4)) & 15u;
                D += ((int)(nib | (((qh >> l) & 1u) << 4)) - 16) * (int)xq[32 * u + l];
            }
            acc += s_of(sc, u) * (f16_at(blk) * (float)D);
        } else if constexpr (TYPE == AH_GGML_Q4_K) {
            const uint8_t *sb = row + 144 * u;
            const float d = f16_at(sb), dmin = f16_at(sb + 2);
            for (uint32_t j = 0; j < 8 && 256 * u + 32 * j < n_in; ++j) {
                // get_scale_min_k4 (format/quant.rs:200-213)
                const uint8_t *s12 = sb + 4;
                uint32_t scj, mj;
                if (j < 4) {
                    scj = byte_at(s12, j) & 63;
                    mj = byte_at(s12, j + 4) & 63;
                } else {
                    scj = (byte_at(s12, j + 4) & 15) | ((byte_at(s12, j - 4) >> 6) << 4);
                    mj = (byte_at(s12, j + 4) >> 4) | ((byte_at(s12, j) >> 6) << 4);
                }
                int D = 0, X = 0;
                for (uint32_t l = 0; l < 32; ++l) {
                    const uint32_t k = 256 * u + 32 * j + l;
                    if (k >= n_in) break;
                    const int q = (int)((byte_at(sb + 16, 32 * (j / 2) + l) >> (4 * (j & 1))) & 15);
                    D += q * (int)xq[k];
                    X += (int)xq[k];
                }
                acc += s_of(sc, 8 * u + j) * ((d * (float)scj) * (float)D - (dmin * (float)mj) * (float)X);
            }
        } else if constexpr (TYPE == AH_GGML_Q2_K || TYPE == AH_GGML_Q3_K) {
            // element 16g + l of the super-block is bit pair r of the qs byte 32n + 16p + l, with
            // g = 8n + 2r + p (format/quant.rs:308-476); Q3_K adds bit 4n + r of hmask[16p + l]
            // as the code's third bit and subtracts 4
            constexpr bool Q3 = TYPE == AH_GGML_Q3_K;
            const uint8_t *sb = row + (Q3 ? 110u : 84u) * u;
            const float d = Q3 ? f16_at(sb + 108) : f16_at(sb + 80), dmin = Q3 ? 0.0f : f16_at(sb + 82);
            for (uint32_t g = 0; g < 16 && 256 * u + 16 * g < n_in; ++g) {
                const uint32_t n = g / 8, r = (g % 8) / 2, pp = g % 2;
                int D = 0, X = 0;
                for (uint32_t l = 0; l < 16; ++l) {
                    const uint32_t k = 256 * u + 16 * g + l;
                    if (k >= n_in) break;
                    int q = (int)((byte_at(sb + (Q3 ? 32 : 16), 32 * n + 16 * pp + l) >> (2 * r)) & 3u);
                    if (Q3) q = (q | (int)(((byte_at(sb, 16 * pp + l) >> (4 * n + r)) & 1u) << 2)) - 4;
                    D += q * (int)xq[k];
                    X += (int)xq[k];
                }
                const float S = s_of(sc, (256 * u + 16 * g) / 32);
                if constexpr (Q3) {
                    const uint32_t j = g % 8, hi = j / 4, i = j % 4;
                    const uint32_t av = byte_at(sb + 96, 4 * hi + i), tv = byte_at(sb + 104, i);
                    const int scg = (int)(((av >> (4 * n)) & 15u) | (((tv >> (4 * n + 2 * hi)) & 3u) << 4)) - 32;
                    acc += S * ((d * (float)scg) * (float)D);
                } else {
                    const uint32_t sv = byte_at(sb, g);
                    acc += S * ((d * (float)(sv & 15u)) * (float)D - (dmin * (float)(sv >> 4)) * (float)X);
                }
            }
        } else {  // Q6_K: element 128n + 32t + l (format/quant.rs:556-599), 16-groups g
            const uint8_t *sb = row + 210 * u;
            const float d = f16_at(sb + 208);
            for (uint32_t g = 0; g < 16 && 256 * u + 16 * g < n_in; ++g) {
                int D = 0;
                for (uint32_t i = 0; i < 16; ++i) {
                    const uint32_t e = 16 * g + i, k = 256 * u + e;
                    if (k >= n_in) break;
                    const uint32_t n = e / 128, t = (e % 128) / 32, l = e % 32;
                    const uint32_t lb = byte_at(sb, 64 * n + l + 32 * (t & 1));
                    const uint32_t hb = byte_at(sb + 128, 32 * n + l);
                    const int uq = (int)(((t < 2 ? lb : lb >> 4) & 15) | (((hb >> (2 * t)) & 3) << 4));
                    D += (uq - 32) * (int)xq[k];
                }
                const int scg = (int)(int8_t)byte_at(sb + 192, g);
                acc += s_of(sc, (256 * u + 16 * g) / 32) * ((d * (float)scg) * (float)D);
            }
        }
    }
    return acc;
}

// The exact path at speed: the flagged tokens of a workgroup tile through the streaming GEMV's
// dot units (exact v_dot4 group dots folded in f32 with the token's own block scales, so no band
// applies; the same arithmetic as a decode GEMV of that token).  The loop is uniform over the
// workgroup: `fm` holds the tile's flagged tokens (bit tl) alike in every wave, and every wave
// calls this.  Per batch of up to kBatch tokens and per window of kWin 32-blocks of the split's
// K range, the workgroup's threads stage each token's codes, block scales and code sums in LDS
// (`win`: the MFMA operand ring or planes, free once every wave is past its loop) in the GEMV's
// layout, shifted so the units index it by absolute block; then lane (j, h) of each wave takes
// row row_w + 32 n + j, the two lane halves alternating units, reading the weights from the GGUF
// rows in memory once for the whole batch.  A unit whose reads could pass the tensor's end (the
// units read up to a dword past their bytes; the tail of a caller-wrapped payload), or any unit
// of a payload whose start is not 16-byte aligned, takes exact_row.  Partials (scaled == false)
// are stored in the reduction's units, divided by the token scale.
namespace xp {
constexpr uint32_t kWin = 64;   // 32-blocks per staged window (2048 K; 3.2 KB of LDS per token)
constexpr uint32_t kBatch = 8;  // flagged tokens staged at once, LDS permitting
constexpr uint32_t kWinBytes = kWin * 32 + kWin * 32 / 16 + kWin * 4 + kWin * 4 + kWin * 2 * 4;
// unit count per 32-block group of a family's GEMV unit, and the unit's bytes
template <int TYPE> constexpr uint32_t unit_blocks() {
    return ah_blk32(TYPE) ? 1u : TYPE == AH_GGML_Q4_K ? 8u : 4u;
}
template <int TYPE> constexpr uint32_t unit_bytes() {
    return TYPE == AH_GGML_Q8_0 ? 34u : TYPE == AH_GGML_Q5_0 ? 22u : TYPE == AH_GGML_Q4_K ? 144u
         : TYPE == AH_GGML_Q6_K ? 210u : TYPE == AH_GGML_Q2_K ? 84u : 110u;  // (super-block bytes)
}
// GEMV unit v of the row at byte `roff` of the tensor `w` (Q8_0 / Q5_0 blocks, Q4_K super-blocks,
// Q6_K / Q2_K / Q3_K half super-blocks), read from global memory.  The units realign their words
// from the byte offset itself, so `w` is passed with the row's offset: only `w` must be aligned
// (16 bytes; Q4_K rows are multiples of 16).
template <int TYPE>
AH_DEV float unit(const uint8_t *w, uint32_t roff, uint32_t v, uint32_t n_in, const ActLds &A) {
    if constexpr (TYPE == AH_GGML_Q8_0) return unit_q8<false>(w, roff + 34u * v, v, A, nullptr);
    else if constexpr (TYPE == AH_GGML_Q5_0) return unit_q5<false>(w, roff + 22u * v, v, A, nullptr);
    else if constexpr (TYPE == AH_GGML_Q4_K) return unit_q4<false>(w, roff + 144u * v, v, n_in, A, nullptr);
    else if constexpr (TYPE == AH_GGML_Q6_K)
        return unit_q6<false>(w, roff + 210u * (v >> 1), v >> 1, v & 1u, n_in, A, nullptr);
    else return unit_k23<TYPE, false>(w, roff + unit_bytes<TYPE>() * (v >> 1), v >> 1, v & 1u, n_in, A, nullptr);
}
}  // namespace xp

template <int TYPE, int NN>
AH_DEV void exact_tokens(const GemmArgs &a, const GemmPartArgs &pa, uint8_t *win, uint32_t win_bytes, uint64_t fm0,
                         uint64_t fm1, uint32_t tok_base, uint32_t row_w, uint32_t tok_lo, uint32_t tok_hi,
                         float *ybase, bool scaled, uint32_t u_lo, uint32_t u_hi) {
    const uint32_t lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
    const uint32_t nb32 = (a.n_in + 31) / 32;
    // the split's K range in 32-blocks, and in GEMV units (halves for Q6_K / Q2_K / Q3_K)
    constexpr bool kHalves = !ah_blk32(TYPE) && TYPE != AH_GGML_Q4_K;
    const uint32_t b_lo = ah_blk32(TYPE) ? u_lo : 8u * u_lo;
    const uint32_t b_hi = ah_blk32(TYPE) ? (u_hi < nb32 ? u_hi : nb32) : 8u * u_hi;
    const uint32_t v_lo = kHalves ? 2u * u_lo : u_lo, v_hi = kHalves ? 2u * u_hi : (ah_blk32(TYPE) ? b_hi : u_hi);
    constexpr uint32_t kVB = kHalves ? 4u : xp::unit_blocks<TYPE>();  // 32-blocks per GEMV unit
    const bool aligned = (reinterpret_cast<uintptr_t>(pa.w) & 15u) == 0;
    // tokens per batch: each staged in a window of its own, so that one weight unit read from
    // memory serves every token of the batch (the later reads hit the cache); the lanes' sums per
    // token and row block sit after the windows, one slot per lane (no lane reads another's)
    const uint32_t waves = blockDim.x / 64, wave = threadIdx.x / 64;
    const uint32_t acc_bytes = waves * xp::kBatch * NN * 256u;
    uint32_t nmax = (win_bytes - acc_bytes) / xp::kWinBytes;
    nmax = nmax < xp::kBatch ? nmax : xp::kBatch;
    float *const vacc = reinterpret_cast<float *>(win + win_bytes - acc_bytes) + wave * xp::kBatch * NN * 64u + lane;
    auto vslot = [&](uint32_t i, int n) -> float & { return vacc[(i * NN + (uint32_t)n) * 64u]; };
    uint64_t rest0 = fm0, rest1 = fm1;
    while ((rest0 | rest1) != 0ull) {
        // the batch: up to nmax of the remaining tokens, lowest first (masks over the tile)
        uint64_t bm0 = 0ull, bm1 = 0ull;
        uint32_t nt = 0;
        while (nt < nmax && (rest0 | rest1) != 0ull) {
            if (rest0) {
                bm0 |= rest0 & (0ull - rest0);
                rest0 &= rest0 - 1;
            } else {
                bm1 |= rest1 & (0ull - rest1);
                rest1 &= rest1 - 1;
            }
            ++nt;
        }
        // the batch's tokens in order: (tl, i) for i = 0, 1, ... (i picks the token's window)
        auto for_tokens = [&](auto &&fn) {
            uint32_t i = 0;
            for (uint64_t m = bm0; m; m &= m - 1) fn((uint32_t)__builtin_ctzll(m), i++);
            for (uint64_t m = bm1; m; m &= m - 1) fn(64u + (uint32_t)__builtin_ctzll(m), i++);
        };
        for_tokens([&](uint32_t, uint32_t i) {
#pragma unroll
            for (int n = 0; n < NN; ++n) vslot(i, n) = 0.0f;
        });
        auto act = [&](uint32_t i, uint32_t g0) {  // token i's window, indexed by absolute block
            uint8_t *wb = win + i * xp::kWinBytes;
            ActLds A;
            A.codes = reinterpret_cast<int8_t *>(wb) - pad_k(32u * g0);
            A.fsc = reinterpret_cast<float *>(wb + codes_bytes(32u * xp::kWin)) - g0;
            A.fx32 = A.fsc + xp::kWin;  // (each array shifted by its window's first block)
            A.xs16 = reinterpret_cast<int32_t *>(A.fx32 + g0 + xp::kWin) - 2u * g0;
            return A;
        };
        for (uint32_t g0 = b_lo & ~7u; g0 < b_hi; g0 += xp::kWin) {
            ah_lds_barrier();  // every wave is past its loop (first window) or the last window
            for_tokens([&](uint32_t tl, uint32_t i) {
                const size_t t = (size_t)tok_base + tl;
                const ActLds A = act(i, g0);
                // (whole quads: blockDim is a multiple of 64, and so is 4 kWin)
                for (uint32_t q = threadIdx.x; q < 4u * xp::kWin; q += blockDim.x) {
                    const uint32_t b = g0 + q / 4;
                    const QuadOut o = quad_quant(quad_load(a.fcodes + t * a.n_in, a.fscales + t * nb32, AH_SRC_CODES,
                                                           a.n_in, 0, b, b < nb32),
                                                 AH_SRC_CODES, b, nullptr, 0);
                    store_quad(A, b, o);
                }
            });
            ah_lds_barrier();
            const uint32_t w_lo = v_lo > g0 / kVB ? v_lo : g0 / kVB;
            const uint32_t w_end = (g0 + xp::kWin) / kVB, w_hi = v_hi < w_end ? v_hi : w_end;
#pragma unroll
            for (int n = 0; n < NN; ++n) {
                const uint32_t row = row_w + 32u * n + j;
                if (row >= pa.n_out) continue;
                const uint32_t roff = row * pa.row_bytes;
                for (uint32_t u = w_lo + h; u < w_hi; u += 2) {
                    const uint32_t sb = kHalves ? u >> 1 : u;  // the unit's block / super-block
                    const size_t end = (size_t)roff + (size_t)xp::unit_bytes<TYPE>() * (sb + 1) + 16u;
                    const bool fast = aligned && end <= pa.w_bytes;
                    for_tokens([&](uint32_t tl, uint32_t i) {
                        if (tl < tok_lo || tl >= tok_hi) return;  // another wave's tokens
                        float add = 0.0f;
                        if (fast) add = xp::unit<TYPE>(pa.w, roff, u, a.n_in, act(i, g0));
                        else if (!kHalves || (u & 1u) == 0) {  // a half's super-block once, whole
                            const size_t t = (size_t)tok_base + tl;
                            add = exact_row<TYPE>(pa.w + roff, a.fcodes + t * a.n_in, a.fscales + t * nb32, a.n_in,
                                                  sb, sb + 1, 0);
                        }
                        vslot(i, n) += add;
                    });
                }
            }
        }
        for_tokens([&](uint32_t tl, uint32_t i) {
            if (tl < tok_lo || tl >= tok_hi) return;
            const size_t t = (size_t)tok_base + tl;
            const float ts = ah_ts_value(__builtin_bit_cast(uint32_t, a.tok_scale[t]));
#pragma unroll
            for (int n = 0; n < NN; ++n) {
                const float vi = vslot(i, n);
                const uint32_t row = row_w + 32u * n + j;
                const float sum = vi + __shfl_xor(vi, 32, 64);
                if (h == 0 && row < pa.n_out) {
                    ybase[(size_t)(tl - tok_lo) * pa.n_out + row] = scaled ? sum : sum / ts;
                    if (const uint32_t oc = scaled ? ah_out_code(sum) : 0u)
                        ah_record(a.status, ah_out_key(pa.key0 + (uint64_t)t * pa.n_out + row, oc));
                }
            }
        });
    }
}


// The epilogue of both GEMM designs.  acc[m][n] holds the wave's sums in the 32x32 MFMA D layout
// (token tiles m, 32-row tiles n from row_w); units [u_lo, u_hi) (Q8_0 blocks, K-quant
// super-blocks) are the split's K range, which the exact path of flagged tokens recomputes.
template <int TYPE, int NM, int NN>
AH_DEV __attribute__((always_inline)) void gemm_store(const GemmArgs &a, const GemmPartArgs &pa,
                                                      const f32x16 (&acc)[NM][NN], uint32_t row_w,
                                                      const bool (&rl)[NN], const uint32_t (&rbase)[NN],
                                                      uint32_t tok0, uint32_t ntile, uint32_t split,
                                                      uint32_t u_lo, uint32_t u_hi, uint8_t *win, uint32_t win_bytes) {
    const int lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
    // D layout of a 32x32 MFMA: lane (j, h), register r -> row i = 8*(r/4) + 4*h + (r%4), col j.
    // Token scales (1.0 for partials) are loaded up front; lanes past n_out, tokens past n_tok and
    // flagged tokens (bit 0 of their scale) store out of range, so there is no branch per element.
    // fm[0..1] collect the tile's flagged tokens (bit tl) for the exact path after the stores.
    uint64_t fm[2] = {0ull, 0ull};
    float *ybase = pa.splits == 1 ? pa.y + (size_t)tok0 * pa.n_out
                                  : pa.y + ((size_t)split * a.n_tok + tok0) * pa.n_out;
    const __amdgpu_buffer_rsrc_t ry = ah_rsrc(ybase, ntile * pa.n_out * 4u);
    const __amdgpu_buffer_rsrc_t rt = ah_rsrc(a.tok_scale + tok0, ntile * 4u);
    const bool scaled = pa.splits == 1;
    // outputs the contract refuses (unsplit parts; a split part's reduction checks its sums): the
    // store loop only ORs the compare masks (scalar registers); a rare second pass reads this
    // lane's own stores back (once they are complete, bypassing L1) and records them
    uint64_t obad = 0ull;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        uint32_t sc[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = ah_ld32(rt, 4 * (32 * m + 8 * (r / 4) + 4 * h + (r % 4)));
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            // lanes of half h hold token 32m + 8(r/4) + 4h + r%4
            const uint64_t b = __builtin_amdgcn_ballot_w64(ah_ts_flagged(sc[r]));
            const uint32_t tl0 = 32 * m + 8 * (r / 4) + (r % 4);
            fm[tl0 >> 6] |= (b & 1ull) << (tl0 & 63);
            fm[(tl0 + 4) >> 6] |= ((b >> 32) & 1ull) << ((tl0 + 4) & 63);
        }
#pragma unroll
        for (int n = 0; n < NN; ++n) {
            const uint32_t row = row_w + 32 * n + j;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t tl = 32 * m + 8 * (r / 4) + 4 * h + (r % 4);
                const bool ok = rl[n] && tl < ntile && !ah_ts_flagged(sc[r]);
                const float v = acc[m][n][r] * (scaled ? ah_ts_value(sc[r]) : 1.0f);
                obad |= __builtin_amdgcn_ballot_w64(ok && !(__builtin_fabsf(v) < 0x1p31f));
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry,
                                                      ok ? (tl * pa.n_out + row) * 4u : kOob, 0, 0);
            }
        }
    }
    if (scaled && obad != 0ull) {
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        for (uint32_t e = 0; e < 16u * NM * NN; ++e) {
            const uint32_t m = e / (16 * NN), n = (e / 16) % NN, r = e % 16;
            const uint32_t tl = 32 * m + 8 * (r / 4) + 4 * h + (r % 4), row = row_w + 32 * n + j;
            if (!rl[n] || tl >= ntile || ah_ts_flagged(ah_ld32(rt, 4 * tl))) continue;
            const float v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ry, (tl * pa.n_out + row) * 4u, 0, 1));
            if (const uint32_t oc = ah_out_code(v)) ah_record(a.status, ah_out_key(pa.key0 + (uint64_t)(tok0 + tl) * pa.n_out + row, oc));
        }
    }
    // flagged tokens (the same in every wave: the workgroup's waves share its tokens)
    if ((fm[0] | fm[1]) != 0ull)
        exact_tokens<TYPE, NN>(a, pa, win, win_bytes, fm[0], fm[1], tok0, row_w, 0u, ntile, ybase, scaled, u_lo, u_hi);
}

// The kernel body, on an LDS ring of RG slots of buf_bytes<TYPE> at `lds`.
template <int TYPE, int WV, int RG>
// (by value: with a reference to the kernel argument the Q8_0 kernel grows from 207 to 256 VGPRs)
AH_DEV __attribute__((always_inline)) void gemm_rb_body(GemmArgs a, uint8_t *lds_base) {
    constexpr int NN = rb::kNN, NM = rb::nm<TYPE>(), NW = rb::nw<TYPE, RG>(), DW = rb::dw<TYPE, RG>();
    constexpr int kTok = rb::tok<TYPE>();
    constexpr int kAN = rb::an<TYPE, WV>();
    constexpr int kR = RG;
    static_assert(TYPE != AH_GGML_Q4_K || kR == 4, "the split sums ride with a super-block's last slice");
    constexpr uint32_t kBuf = rb::buf_bytes<TYPE>();
    auto lds = [&](int k) -> uint8_t * { return lds_base + k * kBuf; };
    uint8_t *const xmin_lds = lds_base + kR * kBuf;  // Q4_K split sums of the current super-block
    // XCD-aware order: dispatch i goes to XCD i % 8, so XCD x takes logical ids
    // [x * per, (x + 1) * per).  Consecutive logical ids share a weight row tile and split, so the
    // workgroups reading the same weights share one XCD's L2.  The grid is a multiple of 8.
    const uint32_t per = gridDim.x >> 3;
    const uint32_t L = (blockIdx.x & 7u) * per + (blockIdx.x >> 3);
    if (L >= a.n_wg) return;  // whole workgroup, before any barrier
    // The part owning L.  Q8_0 launches take one part (rb::max_parts): with a runtime part index
    // the compiler turns the slice loads' bounds selects into branches and the Q8_0 kernel grows
    // from 207 to 256 VGPRs and spills.
    uint32_t pi = 0;
#pragma unroll
    for (uint32_t i = 1; i < rb::max_parts<TYPE>(); ++i)
        if (i < a.n_parts && L >= a.p[i].wg_begin) pi = i;
    const GemmPartArgs &pa = a.p[pi];
    const uint32_t Lp = L - pa.wg_begin;
    const uint32_t tt = Lp % pa.tok_tiles, rest = Lp / pa.tok_tiles;
    const uint32_t split = rest % pa.splits, rtile = rest / pa.splits;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, h = lane >> 5;
    const uint32_t row_w = rtile * rb::rows<WV>() + wave * 32 * NN;
    uint32_t rbase[NN];
    bool rl[NN];
#pragma unroll
    for (int n = 0; n < NN; ++n) {
        const uint32_t r = row_w + 32 * n + j;
        rl[n] = r < pa.n_out;
        rbase[n] = (rl[n] ? r : 0u) * pa.row_bytes;
    }
    const uint32_t tok0 = tt * kTok;
    const uint32_t ntile = a.n_tok - tok0 < (uint32_t)kTok ? a.n_tok - tok0 : (uint32_t)kTok;
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(pa.w, pa.w_bytes);
    const __amdgpu_buffer_rsrc_t rx = ah_rsrc(a.xh + (size_t)tok0 * a.kpad, ntile * a.kpad * 2u);
    const uint32_t nsb = a.kpad / 256;
    const __amdgpu_buffer_rsrc_t rm =
        ah_rsrc(TYPE == AH_GGML_Q4_K ? a.xmin + (size_t)tok0 * nsb * 16 : a.xh,
                TYPE == AH_GGML_Q4_K ? ntile * nsb * 32u : 0u);

    // stages: whole super-blocks for the K-quants (zero activations past n_in; their folds are
    // per super-block, at its last stage), pairs for Q8_0
    const uint32_t nstages = !ah_blk32(TYPE) ? a.kpad / kKS : ((a.n_in + 2 * kKS - 1) / (2 * kKS)) * 2;
    const uint32_t st_begin = split * pa.stages_per_split;
    uint32_t st_end = st_begin + pa.stages_per_split;
    if (st_end > nstages) st_end = nstages;

    // The f16 activation slice of a stage (kTok tokens x 64 K) goes global -> LDS directly (no
    // registers), slots - 1 stages ahead.  Wave w's instruction i fills bytes [(w*kAN + i) KB, +1 KB) of
    // the slot, lane l at +16*l: token t = o / 128 at LDS chunk c' = (o / 16) % 8, which holds the
    // token's K chunk c' ^ ((t >> 1) & 7).  The XOR spreads the 32 token rows an MFMA fragment read
    // touches over all 64 banks.  Stages past the split and tokens past the tile read zeros.
    const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
    auto act_dma = [&](uint8_t *buf, uint32_t st) {
        const bool live = st < st_end;
#pragma unroll
        for (int i = 0; i < kAN; ++i) {
            const uint32_t o = (wv * kAN + i) * 1024u + lane * 16u;
            const uint32_t t = o >> 7, c = ((o >> 4) & 7u) ^ ((t >> 1) & 7u);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rx, (__attribute__((address_space(3))) void *)(buf + (wv * kAN + i) * 1024u), 16,
                live && t < ntile ? (t * a.kpad + st * kKS + 8 * c) * 2u : kOob, 0, 0, 0);
        }
    };
    // Q4_K: the 32-byte split code sums of super-block sb for the tile's tokens, issued at the
    // super-block's first stage just before the slice of its last stage, the one that reads them.
    // Wave w, lane l < xlanes: token w * xtok + l / 2, bytes 16 (l & 1) .. +16.
    auto xmin_dma = [&](uint32_t st) {
        if constexpr (TYPE == AH_GGML_Q4_K) {
            constexpr uint32_t kXT = rb::xtok<WV>(), kXL = rb::xlanes<WV>();
            const uint32_t t = wv * kXT + ((uint32_t)lane >> 1);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rm, (__attribute__((address_space(3))) void *)(xmin_lds + wv * 1024u), 16,
                st < st_end && (uint32_t)lane < kXL && t < ntile ? (t * nsb + st / 4) * 32u + 16u * (lane & 1) : kOob,
                0, 0, 0);
        }
    };
    const uint32_t sw = (uint32_t)(j >> 1) & 7u;
    auto frag = [&](const uint8_t *buf, int m, int kk) -> f16x8 {
        return *reinterpret_cast<const f16x8 *>(buf + (m * 32 + j) * (kKS * 2) + 16 * (((uint32_t)kk >> 3) ^ sw));
    };

    f32x16 acc[NM][NN], P[NM][NN];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int n = 0; n < NN; ++n) acc[m][n] = P[m][n] = (f32x16){};
    float fd[NN], fdm[NN];
    uint32_t s0[NN], s1[NN], s2[NN];
#pragma unroll
    for (int n = 0; n < NN; ++n) {
        fd[n] = fdm[n] = 0.0f;
        s0[n] = s1[n] = s2[n] = 0u;
    }

    // Prologue: the loads of three notional stages before st_begin, in the loop's own order (slice,
    // then the weight fetch DW stages ahead of the notional stage; fetches before st_begin are
    // out-of-range dummies), so every stage's wait count is the same compile-time number.
    WRb W[NW];
    auto prologue = [&](auto kc) {
        constexpr int k = decltype(kc)::value, rel = k - (kR - 1) + DW;  // fetched stage - st_begin
        act_dma(lds(k), st_begin + k);
        constexpr int wi = ((rel % NW) + NW) % NW, P = ((rel % 4) + 4) % 4;
        W[wi] = fetch_rb<TYPE, P, NN>(rs, rbase, rl, rel >= 0 ? st_begin + rel : st_begin, a.n_in, h,
                                      rel >= 0 && st_begin + rel < st_end);
    };
    prologue(std::integral_constant<int, 0>{});
    if constexpr (kR > 2) prologue(std::integral_constant<int, 1>{});
    if constexpr (kR > 3) prologue(std::integral_constant<int, 2>{});

    auto stage = [&](auto uc, uint32_t st) {
        constexpr int u = decltype(uc)::value;
        // the slice of this stage is complete in every wave, and every wave is done with the slot
        // the next slice goes to (read by the previous stage)
        ah_vm_lds_barrier<rb::wait_count<TYPE, WV, RG>(u)>();
        if constexpr (u == 0) xmin_dma(st);
        act_dma(lds((u + kR - 1) % kR), st + kR - 1);
        W[(u + DW) % NW] = fetch_rb<TYPE, (u + DW) % 4, NN>(rs, rbase, rl, st + DW, a.n_in, h, st + DW < st_end);
        __builtin_amdgcn_sched_barrier(0);  // the requests above stay ahead of this stage's work
        const uint8_t *cur = lds(u % kR);
        const WRb &wc = W[u % NW];
        if constexpr (ah_blk32(TYPE)) {
            // 2*NM*NN MFMA chains per stage (block bb, token tile m, row tile n), each two MFMAs
            // into a fresh accumulator that is folded with the block's d.  The fold of chain c-1
            // is issued after chain c's MFMAs, so the VALU fold overlaps the matrix core.
            // A block past n_in has zero codes and d = 0 against zero activations.
            float d[2][NN];
            f16x8 bq[2][NN][2];
#pragma unroll
            for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                for (int n = 0; n < NN; ++n) {
                    const u32x4 v = wc.v[2 * n + bb];
                    uint32_t f[8];
                    if constexpr (TYPE == AH_GGML_Q8_0) {
                        const uint32_t blk = rbase[n] + 34 * (st * 2 + bb);
                        const uint32_t shc = (blk + 2 + 16 * h) & 3u;  // 0 or 2
                        const uint32_t w5[5] = {v.x, v.y, v.z, v.w, wc.s[4 * n + 2 * bb]};
                        const uint32_t dw = wc.s[4 * n + 2 * bb + 1];
                        d[bb][n] = ah_f16_bits_to_f32((dw >> (8 * (blk & 3u))) & 0xffffu);
#pragma unroll
                        for (int i = 0; i < 4; ++i) i8x4_to_f16(ah_alignbyte(w5[i + 1], w5[i], shc), f[2 * i], f[2 * i + 1]);
                    } else {
                        // Q5_0 (format/quant.rs:263-297): lane half h takes outputs 16h..16h+15,
                        // the low (h = 0) or high nibbles of qs[0..15] with qh bits 16h.. as the
                        // fifth bit; u - 16 is exact in f16
                        const uint32_t blk = rbase[n] + 22 * (st * 2 + bb);
                        const bool odd = (blk & 3u) != 0;  // the block starts 2 bytes into its first dword
                        const uint32_t w6[6] = {v.x, v.y, v.z, v.w, wc.s[4 * n + 2 * bb], wc.s[4 * n + 2 * bb + 1]};
                        d[bb][n] = ah_f16_bits_to_f32((odd ? w6[0] >> 16 : w6[0]) & 0xffffu);
                        const uint32_t qh = odd ? w6[1] : ah_alignbyte(w6[1], w6[0], 2);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const uint32_t qs = odd ? w6[i + 2] : ah_alignbyte(w6[i + 2], w6[i + 1], 2);
                            const uint32_t nib = (h ? qs >> 4 : qs) & 0x0F0F0F0Fu;
                            const uint32_t hb = (qh >> (16 * h + 4 * i)) & 0xFu;
                            u5x4_to_f16(nib | (((hb * 0x00204081u) & 0x01010101u) << 4), f[2 * i], f[2 * i + 1]);
                        }
                    }
                    bq[bb][n][0] = pack8(f[0], f[1], f[2], f[3]);
                    bq[bb][n][1] = pack8(f[4], f[5], f[6], f[7]);
                }
            constexpr int NC = 2 * NM * NN;
            f32x16 pq[2];
#pragma unroll
            for (int c = 0; c <= NC; ++c) {
                if (c < NC) {
                    const int bb = c / (NM * NN), m = (c / NN) % NM, n = c % NN;
                    const f16x8 a0 = frag(cur, m, 32 * bb + 16 * h), a1 = frag(cur, m, 32 * bb + 16 * h + 8);
                    pq[c & 1] = mfma(a0, bq[bb][n][0], (f32x16){});
                    pq[c & 1] = mfma(a1, bq[bb][n][1], pq[c & 1]);
                }
                if (c > 0) {
                    const int pc = c - 1, bb = pc / (NM * NN), m = (pc / NN) % NM, n = pc % NN;
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[m][n][r] = __builtin_fmaf(d[bb][n], pq[pc & 1][r], acc[m][n][r]);
                }
            }
        } else if constexpr (TYPE == AH_GGML_Q6_K) {
            // Stage u of the super-block: half n = u/2, nibble u&1.  k-step gg is the 16-group
            // G = 4u + gg (one int8 scale); lane half h takes its elements 8h..8h+7, i.e. ql bytes
            // 64n + 16gg + 8h + e, qh bytes 32n + 16(gg&1) + 8h + e at bit 2(2(u&1) + gg/2)
            // (format/quant.rs:556-599).  The group scale splits as sc = 16a + b (a = sc >> 4 in
            // -8..7, b = sc & 15), so a weight's sc*(u-32) is the sum of two exact f16 operands,
            // 16a*(u-32) (a multiple of 16 below 2^12 with at most 9 significant bits) and
            // b*(u-32) (|.| <= 480).  Both go to MFMAs into the super-block accumulator P, and d
            // is folded once per super-block: twice the MFMAs of one operand per group, a
            // sixteenth of the folds.
            const uint32_t sh = (rbase[0] + 210 * (st / 4)) & 3u;  // 0 or 2
            const uint32_t scw = ah_alignbyte(wc.s[1], wc.s[0], sh);
            const uint32_t ql[16] = {wc.v[0].x, wc.v[0].y, wc.v[0].z, wc.v[0].w, wc.v[1].x, wc.v[1].y,
                                     wc.v[1].z, wc.v[1].w, wc.v[2].x, wc.v[2].y, wc.v[2].z, wc.v[2].w,
                                     wc.v[3].x, wc.v[3].y, wc.v[3].z, wc.v[3].w};
            const uint32_t qh[8] = {wc.v[4].x, wc.v[4].y, wc.v[4].z, wc.v[4].w,
                                    wc.v[5].x, wc.v[5].y, wc.v[5].z, wc.v[5].w};
            constexpr int nib = u & 1;
            f16x8 bhi[4], blo[4];
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) {
                uint32_t uu[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t lw = ah_alignbyte(ql[4 * gg + i + 1], ql[4 * gg + i], sh);
                    const uint32_t hw = ah_alignbyte(qh[4 * (gg & 1) + i + 1], qh[4 * (gg & 1) + i], sh);
                    const uint32_t lo4 = nib ? ((lw >> 4) & 0x0F0F0F0Fu) : (lw & 0x0F0F0F0Fu);
                    uu[i] = lo4 | (((hw >> (2 * (2 * nib + gg / 2))) & 0x03030303u) << 4);
                }
                uint32_t f[4];
                u6x4_to_f16(uu[0], f[0], f[1]);
                u6x4_to_f16(uu[1], f[2], f[3]);
                const int sc = (int)(int8_t)((scw >> (8 * gg)) & 0xffu);
                const _Float16 ha = (_Float16)(float)(16 * (sc >> 4)), hb = (_Float16)(float)(sc & 15);
                const f16x2 a2 = {ha, ha}, b2 = {hb, hb};
                bhi[gg] = pack8(as_u(as_h2(f[0]) * a2), as_u(as_h2(f[1]) * a2), as_u(as_h2(f[2]) * a2),
                                as_u(as_h2(f[3]) * a2));
                blo[gg] = pack8(as_u(as_h2(f[0]) * b2), as_u(as_h2(f[1]) * b2), as_u(as_h2(f[2]) * b2),
                                as_u(as_h2(f[3]) * b2));
            }
#pragma unroll
            for (int gg = 0; gg < 4; ++gg)
#pragma unroll
                for (int m = 0; m < NM; ++m) {
                    const f16x8 av = frag(cur, m, 16 * gg + 8 * h);
                    P[m][0] = mfma(av, bhi[gg], P[m][0]);
                    P[m][0] = mfma(av, blo[gg], P[m][0]);
                }
            if constexpr (u == 3) {
                const float fd6 = ah_f16_bits_to_f32((wc.s[2] >> (8 * sh)) & 0xffffu);
#pragma unroll
                for (int m = 0; m < NM; ++m) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[m][0][r] = __builtin_fmaf(fd6, P[m][0][r], acc[m][0][r]);
                    P[m][0] = (f32x16){};
                }
            }
        } else {  // Q4_K, stage u of the super-block: qs chunk u = sub-blocks 2u (low), 2u+1 (high)
            if constexpr (u == 0) {
#pragma unroll
                for (int n = 0; n < NN; ++n) {
                    const u32x4 hd = wc.v[2 * n];
                    fd[n] = ah_f16_bits_to_f32(hd.x & 0xffffu);
                    fdm[n] = ah_f16_bits_to_f32(hd.x >> 16);
                    s0[n] = hd.y;
                    s1[n] = hd.z;
                    s2[n] = hd.w;
                }
            }
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                f16x8 bq[NN][2];
#pragma unroll
                for (int n = 0; n < NN; ++n) {
                    const uint32_t scv = hb ? q4k_scale<2 * u + 1, false>(s0[n], s1[n], s2[n])
                                            : q4k_scale<2 * u, false>(s0[n], s1[n], s2[n]);
                    // Low nibbles (hb = 0): the byte q -> f16 1024 + q, times sc minus 1024 sc.
                    // High nibbles: the byte masked in place is 16 q -> f16 1024 + 16 q, times
                    // sc / 16 minus 64 sc.  Both products are exact: sc / 16 and 64 sc are exact
                    // in f16 and q sc <= 945 is representable, so the fused rounding is exact.
                    const _Float16 sc = (_Float16)(uint16_t)scv;
                    const _Float16 scm = hb ? sc * (_Float16)0.0625f : sc;
                    const _Float16 off = sc * (hb ? (_Float16)(-64.0f) : (_Float16)(-1024.0f));
                    const f16x2 sc2 = {scm, scm}, off2 = {off, off};
                    const u32x4 q = wc.v[2 * n + 1];
                    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
                    uint32_t f[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t nb = qw[i] & (hb ? 0xF0F0F0F0u : 0x0F0F0F0Fu);
                        nib4_times(nb, sc2, off2, f[2 * i], f[2 * i + 1]);
                    }
                    bq[n][0] = pack8(f[0], f[1], f[2], f[3]);
                    bq[n][1] = pack8(f[4], f[5], f[6], f[7]);
                }
#pragma unroll
                for (int m8 = 0; m8 < 2; ++m8)
#pragma unroll
                    for (int m = 0; m < NM; ++m) {
                        const f16x8 av = frag(cur, m, 32 * hb + 16 * h + 8 * m8);
#pragma unroll
                        for (int n = 0; n < NN; ++n) P[m][n] = mfma(av, bq[n][m8], P[m][n]);
                    }
            }
            if constexpr (u == 3) {
                // min term: sum_j m_j * X_j over the super-block as one MFMA with K' = 16:
                // A'[tok][8h+e] = split code sum of sub-block e (hi piece h = 0, lo piece h = 1),
                // B'[8h+e][row] = m_e.
#pragma unroll
                for (int n = 0; n < NN; ++n) {
                    const f16x2 m01 = {(_Float16)(float)q4k_scale<0, true>(s0[n], s1[n], s2[n]),
                                       (_Float16)(float)q4k_scale<1, true>(s0[n], s1[n], s2[n])};
                    const f16x2 m23 = {(_Float16)(float)q4k_scale<2, true>(s0[n], s1[n], s2[n]),
                                       (_Float16)(float)q4k_scale<3, true>(s0[n], s1[n], s2[n])};
                    const f16x2 m45 = {(_Float16)(float)q4k_scale<4, true>(s0[n], s1[n], s2[n]),
                                       (_Float16)(float)q4k_scale<5, true>(s0[n], s1[n], s2[n])};
                    const f16x2 m67 = {(_Float16)(float)q4k_scale<6, true>(s0[n], s1[n], s2[n]),
                                       (_Float16)(float)q4k_scale<7, true>(s0[n], s1[n], s2[n])};
                    const f16x8 bm = pack8(as_u(m01), as_u(m23), as_u(m45), as_u(m67));
#pragma unroll
                    for (int m = 0; m < NM; ++m) {
                        constexpr uint32_t kXT = rb::xtok<WV>();
                        const uint32_t T = 32 * m + j;
                        const f16x8 am = *reinterpret_cast<const f16x8 *>(xmin_lds + (T / kXT) * 1024u + (T % kXT) * 32u + 16u * h);
                        const f32x16 pm = mfma(am, bm, (f32x16){});
                        // the d P pass first (it needs no pm), then the dmin pass: the same two
                        // FMAs per element as one fused chain, while the min MFMA completes
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[m][n][r] = __builtin_fmaf(fd[n], P[m][n][r], acc[m][n][r]);
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[m][n][r] = __builtin_fmaf(-fdm[n], pm[r], acc[m][n][r]);
                        P[m][n] = (f32x16){};
                    }
                }
            }
        }
    };

    for (uint32_t st = st_begin; st < st_end; st += 4) {
        stage(std::integral_constant<int, 0>{}, st);
        stage(std::integral_constant<int, 1>{}, st + 1);
        if (ah_blk32(TYPE) && st + 2 >= st_end) break;  // Q8_0 / Q5_0 splits are whole pairs
        stage(std::integral_constant<int, 2>{}, st + 2);
        stage(std::integral_constant<int, 3>{}, st + 3);
    }
    // the slices requested past the split must land before this workgroup's LDS is released
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");

    const uint32_t u_lo = ah_blk32(TYPE) ? 2 * st_begin : st_begin / 4;
    const uint32_t u_hi = ah_blk32(TYPE) ? 2 * st_end : st_end / 4;
    static_assert(rb::lds_bytes<TYPE, WV, RG>() >= xp::kWinBytes + WV * xp::kBatch * NN * 256u,
                  "the exact path stages a token window and its sums in the ring");
    gemm_store<TYPE, NM, NN>(a, pa, acc, row_w, rl, rbase, tok0, ntile, split, u_lo, u_hi, lds_base,
                             rb::lds_bytes<TYPE, WV, RG>());
}

template <int TYPE, int WV, int RG>
__global__ void __launch_bounds__(64 * WV, TYPE == AH_GGML_Q4_K ? 4 : 2) gemm_rb_kernel(GemmArgs a) {
    __shared__ __align__(16) uint8_t lds[rb::lds_bytes<TYPE, WV, RG>()];
    gemm_rb_body<TYPE, WV, RG>(a, lds);
}

// ---- int8-MFMA design (Q8_0; Q4_K below) ------------------------------------------------------
//
// v_mfma_i32_32x32x32_i8 takes one whole 32-block per MFMA: the activation codes (A, M = 32
// tokens) from LDS, the weight codes (B, N = 32 rows) straight from the GGUF bytes, and gives the
// exact int32 block dot D[tok][row] (|D| <= 32 * 127 * 127 < 2^19).  Each block then needs
// y += D * d_rb * S'_tb per element, where S' = 2^(e_b - E_tok) is the block's power-of-two
// activation factor relative to the token's largest block (the token scale 2^(E_tok - 32) is
// applied once at the end, as in the f16 design).  A VALU multiply per element would make that
// fold three VALU operations per element and block.  Instead a second MFMA forms the product
// table as an outer product: v_mfma_f32_32x32x8_bf16 with A'[tok] = (S', S') and B'[row] =
// (d_hi, d_lo), the f16 d split exactly into two bf16 (its top 8 and low 3 significant bits).  S'
// is an exact bf16 whatever the exponent gap (bf16 has the f32 exponent range, so this design has
// no f16 band and flags no token for it).  P = d_hi S' + d_lo S' = d * S' exactly in f32, in the
// same D layout as the int32 dots, and the fold is one convert and one FMA per element and block.
//
// Bounds per 32-block and 32x32 tile: two MFMAs on the matrix core (the int8 one at twice the f16
// rate) against 32 VALU instructions of 64 lanes (4 cycles each): the VALU bounds this design at
// about 128 cycles per 65536 int8 operations a SIMD, a quarter of the int8 MFMA peak.
//
// Q4_K takes the same tiles with a stage of half a super-block (four 32-element sub-blocks): the
// int8 MFMA dots the raw nibbles (0..15) of each sub-block, and the fold per sub-block is
// y += D * (S' d sc_j) - (S' X_j) (dmin m_j), X_j the token's code sum of the sub-block.  Both
// products come from bf16 outer-product MFMAs: d sc_j and dmin m_j (an f16 times a 6-bit integer,
// at most 17 significant bits) split exactly into three bf16 each, S' as one bf16 and S' X_j (at
// most 12 significant bits) as two, hi and lo, which the operand pass writes beside the block
// factors.  The scale product is exact; the min product rounds once in the MFMA's f32 sum.  The
// fold is one convert, one FMA and one subtract per element and sub-block.
//
// Tiling: W waves, each owning 32 weight rows and the workgroup's 128 tokens (4 token tiles); a
// stage is 4 blocks (K = 128).  The stage's activation codes (128 tokens x 128 B, chunk-XOR
// swizzled like the f16 slice) and block factors (128 tokens x 16 B) go global -> LDS into a ring
// of 3 slots, two stages ahead; each wave reads its rows' weight bytes a stage ahead into
// registers.  Every stage issues its weight loads, then its slice: the top of a stage waits for
// vmcnt <= one stage's slice instructions, which completes the stage's slice and its weights.
namespace i8 {
constexpr uint32_t kTok = 128, kKS = 128, kR = 3;
constexpr uint32_t kAct = kTok * kKS;       // activation codes of a slot
constexpr uint32_t kSlot = kAct + 4096;     // + block factors (one 1 KB load per wave)
// Q4_K also stages the tokens' scaled block code sums (one more 1 KB load per wave)
template <int TYPE> constexpr uint32_t slot_bytes() { return kSlot + (TYPE == AH_GGML_Q4_K ? 4096u : 0u); }
template <int TYPE> constexpr int side_loads() { return TYPE == AH_GGML_Q4_K ? 2 : 1; }
template <int W> constexpr int an() { return (int)(kAct / 1024) / W; }
template <int TYPE, int W> constexpr int wait_count() { return (int)(kR - 2) * (an<W>() + side_loads<TYPE>()); }
constexpr uint32_t stages(uint32_t n_in) { return ((n_in + 31) / 32 + 3) / 4; }
}  // namespace i8

typedef int v4i8x4 __attribute__((ext_vector_type(4)));     // 16 int8 codes
typedef int v16i32 __attribute__((ext_vector_type(16)));
typedef short v4bf16 __attribute__((ext_vector_type(4)));   // 4 bf16 bit patterns

// v = a + b + c exactly as three bf16 (the top 8 significant bits, the next 8, the rest), for an
// f32 of at most 24 significant bits whose remainder after 16 fits a bf16 (here d sc and dmin m:
// an f16 times a 6-bit integer, at most 17 bits); the slots [a, b, c, 0] of a bf16 MFMA operand.
AH_DEV v4bf16 bf16x3(float v) {
    const uint32_t a = __builtin_bit_cast(uint32_t, v) & 0xffff0000u;
    const float r = v - __builtin_bit_cast(float, a);  // exact: the bits below a's
    const uint32_t b = __builtin_bit_cast(uint32_t, r) & 0xffff0000u;
    const uint32_t c = __builtin_bit_cast(uint32_t, r - __builtin_bit_cast(float, b)) & 0xffff0000u;
    return __builtin_bit_cast(v4bf16, (u32x2){(a >> 16) | b, c >> 16});
}

template <int TYPE, int W>
__global__ void __launch_bounds__(64 * W, 2) gemm_i8_kernel(GemmArgs a) {
    static_assert(TYPE == AH_GGML_Q8_0 || TYPE == AH_GGML_Q4_K, "the int8 design serves Q8_0 and Q4_K");
    constexpr bool Q4 = TYPE == AH_GGML_Q4_K;
    constexpr int NM = 4, AN = i8::an<W>();
    constexpr uint32_t TPW = i8::kTok / W;  // tokens whose block factors one wave loads
    constexpr uint32_t kSlotB = i8::slot_bytes<TYPE>();
    __shared__ __align__(16) uint8_t lds[i8::kR * kSlotB];
    const uint32_t per = gridDim.x >> 3;  // XCD-aware order, as gemm_rb_body
    const uint32_t L = (blockIdx.x & 7u) * per + (blockIdx.x >> 3);
    if (L >= a.n_wg) return;
    const GemmPartArgs &pa = a.p[0];  // one part per launch
    const uint32_t tt = L % pa.tok_tiles, rest = L / pa.tok_tiles;
    const uint32_t split = rest % pa.splits, rtile = rest / pa.splits;
    const int tid = threadIdx.x, lane = tid & 63, j = lane & 31, h = lane >> 5;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t row_w = rtile * 32u * W + wv * 32u;
    bool rl[1];
    uint32_t rbase[1];
    rl[0] = row_w + j < pa.n_out;
    rbase[0] = (rl[0] ? row_w + j : 0u) * pa.row_bytes;
    const uint32_t tok0 = tt * i8::kTok;
    const uint32_t ntile = a.n_tok - tok0 < i8::kTok ? a.n_tok - tok0 : i8::kTok;
    const uint32_t nbp = a.kpad / 32, nb32 = (a.n_in + 31) / 32;
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(pa.w, pa.w_bytes);
    const __amdgpu_buffer_rsrc_t rx = ah_rsrc(a.xc + (size_t)tok0 * a.kpad, ntile * a.kpad);
    const __amdgpu_buffer_rsrc_t rp = ah_rsrc(a.xsp + (size_t)tok0 * nbp, ntile * nbp * 4u);
    const __amdgpu_buffer_rsrc_t rq = ah_rsrc(Q4 ? a.xsx + (size_t)tok0 * nbp : a.xsp, Q4 ? ntile * nbp * 4u : 0u);
    const uint32_t nstages = i8::stages(a.n_in);
    const uint32_t st_begin = split * pa.stages_per_split;
    const uint32_t st_end = st_begin + pa.stages_per_split < nstages ? st_begin + pa.stages_per_split : nstages;

    auto slot = [&](uint32_t k) -> uint8_t * { return lds + k * kSlotB; };
    // slice of stage st: wave w's instruction i fills slot bytes [(w*AN + i) KB, +1 KB), lane l at
    // +16 l: token t = o / 128 at LDS chunk (o / 16) % 8, which holds the token's K chunk
    // ((o / 16) % 8) ^ ((t >> 1) & 7); then its block factors, lanes < TPW taking tokens w*TPW + l
    auto dma = [&](uint8_t *buf, uint32_t st) {
        const bool live = st < st_end;
#pragma unroll
        for (int i = 0; i < AN; ++i) {
            const uint32_t o = (wv * AN + i) * 1024u + lane * 16u;
            const uint32_t t = o >> 7, c = ((o >> 4) & 7u) ^ ((t >> 1) & 7u);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rx, (__attribute__((address_space(3))) void *)(buf + (wv * AN + i) * 1024u), 16,
                live && t < ntile ? t * a.kpad + st * i8::kKS + 16 * c : kOob, 0, 0, 0);
        }
        const uint32_t t = wv * TPW + lane;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rp, (__attribute__((address_space(3))) void *)(buf + i8::kAct + wv * 1024u), 16,
            live && lane < TPW && t < ntile ? (t * nbp + 4 * st) * 4u : kOob, 0, 0, 0);
        if constexpr (Q4)  // the tokens' scaled code sums of the stage's four blocks, the same way
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rq, (__attribute__((address_space(3))) void *)(buf + i8::kSlot + wv * 1024u), 16,
                live && lane < TPW && t < ntile ? (t * nbp + 4 * st) * 4u : kOob, 0, 0, 0);
    };
    // weight bytes of stage st for row j: per block the lane half's 16 codes (4-aligned window
    // plus the dword after it) and, for half 0, the dword holding d
    struct Wt {
        u32x4 v[4];
        uint32_t s[4], d[4];
    };
    // Q4_K: a stage is half a super-block (sub-blocks 4 (st & 1) .. + 3, pairs 2 (st & 1) and
    // 2 (st & 1) + 1): v[0] = the super-block's header (d, dmin, the 12 scale bytes), v[1] / v[2]
    // = the lane half's 16 qs bytes of the two pairs (low nibbles: the pair's first sub-block)
    auto fetch = [&](uint32_t st) -> Wt {
        Wt f;
        const bool live = st < st_end && rl[0];
        if constexpr (Q4) {
            const uint32_t sb = rbase[0] + 144u * (st >> 1), p0 = 2u * (st & 1u);
            f.v[0] = ah_ld128(rs, live ? sb : kOob);
            f.v[1] = ah_ld128(rs, live ? sb + 16u + 32u * p0 + 16u * h : kOob);
            f.v[2] = ah_ld128(rs, live ? sb + 48u + 32u * p0 + 16u * h : kOob);
            return f;
        }
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            const uint32_t b = 4 * st + bb;
            const bool m = live && b < nb32;
            const uint32_t blk = rbase[0] + 34 * b, c = (blk + 2 + 16 * h) & ~3u;
            f.v[bb] = ah_ld128(rs, m ? c : kOob);
            f.s[bb] = ah_ld32(rs, m ? c + 16 : kOob);
            f.d[bb] = ah_ld32(rs, m && h == 0 ? blk & ~3u : kOob);
        }
        return f;
    };

    f32x16 acc[NM][1];
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[m][0] = (f32x16){};
    const uint32_t sw = (uint32_t)(j >> 1) & 7u;
    auto compute = [&](const uint8_t *buf, const Wt &f, uint32_t st) {
        v4i8x4 A[4];
        v4bf16 Dp[4];
        if constexpr (Q4) {
            // Per sub-block j: the int8 MFMA gives the exact dots D of the codes q (0..15) and the
            // token's codes; the fold is acc += D (2^(e - E) d sc_j) - (2^(e - E) X) (dmin m_j),
            // both products formed exactly-split by a bf16 MFMA as outer products: the token
            // side 2^(e - E) (one bf16) and 2^(e - E) X (two, hi and lo, the operand pass's xsx),
            // the row side d sc_j and dmin m_j (at most 17 bits: three bf16 each, bf16x3).
            const u32x4 hd = f.v[0];
            const uint32_t par = st & 1u;
            const float d = ah_f16_bits_to_f32(hd.x & 0xffffu), dmin = ah_f16_bits_to_f32(hd.x >> 16);
            const uint32_t scw = par ? (hd.w & 0x0F0F0F0Fu) | ((hd.y >> 2) & 0x30303030u) : hd.y & 0x3F3F3F3Fu;
            const uint32_t mw = par ? ((hd.w >> 4) & 0x0F0F0F0Fu) | ((hd.z >> 2) & 0x30303030u) : hd.z & 0x3F3F3F3Fu;
            v4bf16 Mp[4];
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                const u32x4 q = f.v[1 + (bb >> 1)];
                const uint32_t sh = (bb & 1) ? 4u : 0u;
                A[bb] = (v4i8x4){(int)((q.x >> sh) & 0x0F0F0F0Fu), (int)((q.y >> sh) & 0x0F0F0F0Fu),
                                 (int)((q.z >> sh) & 0x0F0F0F0Fu), (int)((q.w >> sh) & 0x0F0F0F0Fu)};
                const float ds = d * (float)((scw >> (8 * bb)) & 0xffu);
                const float dm = dmin * (float)((mw >> (8 * bb)) & 0xffu);
                Dp[bb] = h ? (v4bf16){0, 0, 0, 0} : bf16x3(ds);  // the scale's slots: K 0..3 only
                Mp[bb] = bf16x3(dm);                             // the min's: K 0..3 and 4..7
            }
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const uint32_t t = 32 * m + j;
                const u32x4 sv = *reinterpret_cast<const u32x4 *>(buf + i8::kAct + (t / TPW) * 1024u + (t % TPW) * 16u);
                const u32x4 xv = *reinterpret_cast<const u32x4 *>(buf + i8::kSlot + (t / TPW) * 1024u + (t % TPW) * 16u);
                const uint32_t s4[4] = {sv.x, sv.y, sv.z, sv.w}, x4[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) {
                    const v4i8x4 B = *reinterpret_cast<const v4i8x4 *>(buf + t * i8::kKS + 16 * ((uint32_t)(2 * bb + h) ^ sw));
                    const v16i32 D = __builtin_amdgcn_mfma_i32_32x32x32_i8(B, A[bb], (v16i32){}, 0, 0, 0);
                    // token factor f in K slots 0..2 (half 0); the scaled code sum's hi piece in
                    // slots 0..2 and its lo piece in slots 4..6
                    const uint32_t fb = s4[bb] & 0xffffu, xb = h ? x4[bb] >> 16 : x4[bb] & 0xffffu;
                    const u32x2 sp = {h ? 0u : fb | (fb << 16), h ? 0u : fb};
                    const u32x2 xp2 = {xb | (xb << 16), xb};
                    const f32x16 P = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(__builtin_bit_cast(v4bf16, sp), Dp[bb], (f32x16){}, 0, 0, 0);
                    const f32x16 Pm = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(__builtin_bit_cast(v4bf16, xp2), Mp[bb], (f32x16){}, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[m][0][r] = __builtin_fmaf((float)D[r], P[r], acc[m][0][r]) - Pm[r];
                }
            }
            return;
        }
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            const uint32_t blk = rbase[0] + 34 * (4 * st + bb);
            const uint32_t shc = (blk + 2 + 16 * h) & 3u;  // 0 or 2
            const uint32_t w5[5] = {f.v[bb].x, f.v[bb].y, f.v[bb].z, f.v[bb].w, f.s[bb]};
            A[bb] = (v4i8x4){(int)ah_alignbyte(w5[1], w5[0], shc), (int)ah_alignbyte(w5[2], w5[1], shc),
                             (int)ah_alignbyte(w5[3], w5[2], shc), (int)ah_alignbyte(w5[4], w5[3], shc)};
            // d = d_hi + d_lo exactly: d_hi keeps the top 8 significant bits (an f32 with a zero
            // low half is a bf16), d_lo the other 3 (half 1 loaded d = 0: a zero operand)
            const float d = ah_f16_bits_to_f32((f.d[bb] >> (8 * (blk & 3u))) & 0xffffu);
            const uint32_t hi = __builtin_bit_cast(uint32_t, d) & 0xffff0000u;
            const uint32_t lo = __builtin_bit_cast(uint32_t, d - __builtin_bit_cast(float, hi));
            const u32x2 pr = {(hi >> 16) | (lo & 0xffff0000u), 0u};
            Dp[bb] = __builtin_bit_cast(v4bf16, pr);
        }
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const uint32_t t = 32 * m + j;
            const u32x4 sv = *reinterpret_cast<const u32x4 *>(buf + i8::kAct + (t / TPW) * 1024u + (t % TPW) * 16u);
            const uint32_t s4[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                const v4i8x4 B = *reinterpret_cast<const v4i8x4 *>(buf + t * i8::kKS + 16 * ((uint32_t)(2 * bb + h) ^ sw));
                // tokens on the MFMA's M side, rows on N: the D layout gemm_store reads
                const v16i32 D = __builtin_amdgcn_mfma_i32_32x32x32_i8(B, A[bb], (v16i32){}, 0, 0, 0);
                const u32x2 sp = {h ? 0u : s4[bb], 0u};
                const f32x16 P = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(__builtin_bit_cast(v4bf16, sp), Dp[bb], (f32x16){}, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[m][0][r] = __builtin_fmaf((float)D[r], P[r], acc[m][0][r]);
            }
        }
    };

    Wt F0 = fetch(st_begin), F1;
    __builtin_amdgcn_sched_barrier(0);
    dma(slot(0), st_begin);
    dma(slot(1), st_begin + 1);
    __builtin_amdgcn_sched_barrier(0);
    uint32_t k = 0;  // slot of the current stage
    for (uint32_t st = st_begin; st < st_end; st += 2) {
        ah_vm_lds_barrier<i8::wait_count<TYPE, W>()>();  // slice st (and weights st) landed; slot k+2 free
        F1 = fetch(st + 1);
        __builtin_amdgcn_sched_barrier(0);
        dma(slot(k == 0 ? 2u : k - 1), st + 2);
        __builtin_amdgcn_sched_barrier(0);
        compute(slot(k), F0, st);
        k = k == 2 ? 0u : k + 1;
        if (st + 1 >= st_end) break;
        ah_vm_lds_barrier<i8::wait_count<TYPE, W>()>();
        F0 = fetch(st + 2);
        __builtin_amdgcn_sched_barrier(0);
        dma(slot(k == 0 ? 2u : k - 1), st + 3);
        __builtin_amdgcn_sched_barrier(0);
        compute(slot(k), F1, st + 1);
        k = k == 2 ? 0u : k + 1;
    }
    // the slices requested past the split must land before this workgroup's LDS is released
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    static_assert(i8::kR * kSlotB >= xp::kWinBytes + 4 * xp::kBatch * 256u,
                  "the exact path stages a token window and its sums in the slots");
    // the split's K range in the exact path's units: Q8_0 blocks, Q4_K super-blocks (splits are
    // whole super-blocks: two stages)
    gemm_store<TYPE, NM, 1>(a, pa, acc, row_w, rl, rbase, tok0, ntile, split, Q4 ? st_begin / 2 : 4 * st_begin,
                            Q4 ? (st_end + 1) / 2 : 4 * st_end, lds, i8::kR * kSlotB);
}

// Q4_K and Q6_K parts of one input in one grid (4 waves, 4 slots sized for the larger type):
// each workgroup runs its part's body, a branch uniform over the workgroup.  A group's runs of
// the two types (q/k beside v) then share the CUs one run alone leaves idle.
__global__ void __launch_bounds__(256, 2) gemm_rb_kquant_kernel(GemmArgs a) {
    // the larger of the two bodies' LDS (the Q4_K ring and its split-sum region fit in Q6_K's ring)
    constexpr int kL4 = rb::lds_bytes<AH_GGML_Q4_K, 4, 4>(), kL6 = rb::lds_bytes<AH_GGML_Q6_K, 4, 4>();
    __shared__ __align__(16) uint8_t lds[kL4 > kL6 ? kL4 : kL6];
    const uint32_t per = gridDim.x >> 3;
    const uint32_t L = (blockIdx.x & 7u) * per + (blockIdx.x >> 3);
    if (L >= a.n_wg) return;
    uint32_t pi = 0;
#pragma unroll
    for (uint32_t i = 1; i < kGemmMaxParts; ++i)
        if (i < a.n_parts && L >= a.p[i].wg_begin) pi = i;
    if (a.p[pi].type == AH_GGML_Q4_K) gemm_rb_body<AH_GGML_Q4_K, 4, 4>(a, lds);
    else gemm_rb_body<AH_GGML_Q6_K, 4, 4>(a, lds);
}

// y[tok][row] = tok_scale[tok] * sum_s partial[s][tok][row], summed in split order from 0, for
// every split part of a grouped call in one launch.  A work item is 4 consecutive outputs (VEC:
// every part has n % 4 == 0 and 16-byte aligned planes) or one; a thread issues the loads of 8
// splits before the first add.
constexpr uint32_t kReduceBatch = 8;
constexpr uint32_t kReduceMaxParts = 8;
struct ReducePart {
    const float *part;
    float *y;
    uint64_t begin;  // first work item of the part
    uint64_t key0;   // added to the part's output refusal keys
    uint32_t n_out, splits;
};
struct ReduceArgs {
    ReducePart p[kReduceMaxParts];
    const float *tok_scale;
    unsigned long long *status;
    uint64_t total;  // work items over all parts
    uint32_t n_parts, n_tok;
};
typedef float f32x4 __attribute__((ext_vector_type(4)));
AH_DEV float ts_at(const float *ts, size_t i) { return ah_ts_value(__builtin_bit_cast(uint32_t, ts[i])); }
template <bool VEC>
__global__ void splitk_reduce(ReduceArgs r) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < r.total;
         i += (uint64_t)gridDim.x * blockDim.x) {
        ReducePart P = r.p[0];
#pragma unroll
        for (uint32_t k = 1; k < kReduceMaxParts; ++k)
            if (k < r.n_parts && i >= r.p[k].begin) P = r.p[k];
        const uint64_t li = i - P.begin;
        const size_t n = (size_t)r.n_tok * P.n_out;
        if constexpr (VEC) {
            const size_t n4 = n / 4;
            const f32x4 *p = reinterpret_cast<const f32x4 *>(P.part) + li;
            f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
            for (uint32_t z = 0; z < P.splits; z += kReduceBatch) {
                f32x4 v[kReduceBatch];
#pragma unroll
                for (uint32_t j = 0; j < kReduceBatch; ++j)
                    if (z + j < P.splits) v[j] = __builtin_nontemporal_load(p + (z + j) * n4);
#pragma unroll
                for (uint32_t j = 0; j < kReduceBatch; ++j)
                    if (z + j < P.splits) s += v[j];
            }
            const size_t e = 4 * li;
            f32x4 o;
            o.x = s.x * ts_at(r.tok_scale, e / P.n_out);
            o.y = s.y * ts_at(r.tok_scale, (e + 1) / P.n_out);
            o.z = s.z * ts_at(r.tok_scale, (e + 2) / P.n_out);
            o.w = s.w * ts_at(r.tok_scale, (e + 3) / P.n_out);
            reinterpret_cast<f32x4 *>(P.y)[li] = o;
            const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
            for (int c = 0; c < 4; ++c)
                if (const uint32_t oc = ah_out_code(ov[c])) { ah_record(r.status, ah_out_key(P.key0 + e + c, oc)); break; }
        } else {
            float s = 0.0f;
            for (uint32_t z = 0; z < P.splits; z += kReduceBatch) {
                float v[kReduceBatch];
#pragma unroll
                for (uint32_t j = 0; j < kReduceBatch; ++j)
                    if (z + j < P.splits) v[j] = __builtin_nontemporal_load(P.part + (z + j) * n + li);
#pragma unroll
                for (uint32_t j = 0; j < kReduceBatch; ++j)
                    if (z + j < P.splits) s += v[j];
            }
            P.y[li] = s * ts_at(r.tok_scale, li / P.n_out);
            if (const uint32_t oc = ah_out_code(P.y[li])) ah_record(r.status, ah_out_key(P.key0 + li, oc));
        }
    }
}


// ---- dequantize-once design (gemm_dq_kernel) --------------------------------------------------
//
// The register-blocked kernel above converts every weight fragment once per wave that uses it, so
// its dequantization is paid once per 32- or 64-token tile.  Here a workgroup covers 128 weight
// rows x 128 tokens with 4 waves in a 2 x 2 grid (each wave 64 rows x 64 tokens: 2 x 2 MFMA
// tiles).  Every stage of 64 K the workgroup's 256 threads read the stage's raw GGUF bytes of the
// 128 rows with coalesced loads, convert each weight once to its exact f16 operand and write it
// to an LDS plane [128 rows][64 K]; the activation slice [128 tokens][64 K] comes global -> LDS
// by direct loads.  Waves then read both operands as MFMA fragments (1 KB of LDS per MFMA).  The
// conversion is paid once per 128 tokens and is independent of the MFMA layout, so every GGUF
// family only needs its own stage decoder.  Both planes are double-buffered: while the waves
// multiply stage s, the threads convert stage s + 1 into the other buffer and the loads of the
// stages after it are in flight, so one barrier per stage orders everything.
//
// Operands and exactness are the register-blocked kernel's: the activation is xq * 2^(e_b - E_tok)
// (the operand pass), the Q4_K weight operand sc_j * q, folded with d once per super-block, the
// dmin * m * X term on one extra MFMA per super-block.
namespace dq {
constexpr uint32_t kBM = 128, kBN = 128;
constexpr uint32_t kPlane = 128u * kKS * 2u;  // one [128][64] f16 plane: 16 KB
// Chunk c (8 K values, 16 B) of row r of a [128][64] plane: rows of 128 B, chunks XOR-swizzled
// by (r >> 1) & 7 so that the 32 rows of one fragment read (two chunks each) cover all 64 banks.
AH_DEV uint32_t swz(uint32_t r, uint32_t c) { return r * 128u + 16u * (c ^ ((r >> 1) & 7u)); }

// Super-block bytes and the families this design serves.  Every family's stage (64 K of a row)
// splits the same way over a row's two lane halves h: elements at stage K 16h .. 16h + 15 (the
// "low run") and 32 + 16h .. 32 + 16h + 15 (the "high run"), each from 16 bytes the thread loads.
template <int TYPE> constexpr uint32_t sb_bytes() { return TYPE == AH_GGML_Q4_K ? 144u : TYPE == AH_GGML_Q2_K ? 84u : 110u; }
template <int TYPE> constexpr bool served() { return TYPE == AH_GGML_Q4_K || TYPE == AH_GGML_Q2_K || TYPE == AH_GGML_Q3_K; }

// 16 bytes from a 2-aligned offset (Q3_K blocks are 110 bytes): five dwords realigned.
AH_DEV u32x4 ld16_u2(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    const uint32_t a = off & ~3u, sh = off & 3u;
    const u32x4 v = ah_ld128(rs, a);
    const uint32_t e = ah_ld32(rs, a + 16u);
    return (u32x4){ah_alignbyte(v.y, v.x, sh), ah_alignbyte(v.z, v.y, sh), ah_alignbyte(v.w, v.z, sh), ah_alignbyte(e, v.w, sh)};
}

// This thread's raw bytes of one stage at super-block position P (half n = P >> 1):
//   Q4_K (format/quant.rs:481-510): q = qs[32P + 16h .. +16] (low nibble: sub-block 2P, high:
//        2P + 1); at P = 0 hd = the header (d, dmin, scales[12]).
//   Q2_K (format/quant.rs:308-360): q = qs[32n + 16h .. +16]: element 128n + 32r + 16h + l is bit
//        pair r of byte l, so the stage takes pairs r0 = 2 (P & 1) and r0 + 1; at P = 0 hd = the
//        16 scale bytes (sc low nibble, m high, group g at byte g), x.x = d | dmin << 16.
//   Q3_K (format/quant.rs:362-476): q = qs[32n + 16h .. +16] as Q2_K, x = hmask[16h .. +16] (bit
//        4n + r of byte l is the third bit of element 128n + 32r + 16h + l); at P = 0 hd = the 12
//        scale bytes and d.
struct Raw {
    u32x4 q, x, hd;
};
template <int TYPE, int P>
AH_DEV Raw fetch(__amdgpu_buffer_rsrc_t rs, uint32_t base, uint32_t h, bool live) {
    Raw w;
    w.x = w.hd = (u32x4){0u, 0u, 0u, 0u};
    if constexpr (TYPE == AH_GGML_Q4_K) {
        w.q = ah_ld128(rs, live ? base + 16u + 32u * P + 16u * h : kOob);
        if constexpr (P == 0) w.hd = ah_ld128(rs, live ? base : kOob);
    } else if constexpr (TYPE == AH_GGML_Q2_K) {
        w.q = ah_ld128(rs, live ? base + 16u + 32u * (P >> 1) + 16u * h : kOob);
        if constexpr (P == 0) {
            w.hd = ah_ld128(rs, live ? base : kOob);
            w.x.x = ah_ld32(rs, live ? base + 80u : kOob);
        }
    } else {
        w.q = ld16_u2(rs, live ? base + 32u + 32u * (P >> 1) + 16u * h : kOob);
        w.x = ld16_u2(rs, live ? base + 16u * h : kOob);
        if constexpr (P == 0) w.hd = ld16_u2(rs, live ? base + 96u : kOob);
    }
    return w;
}

// Per-thread scale state of the super-block being converted (from its header).
struct Scales {
    uint32_t w[4];
};
AH_DEV Scales scales_of(const Raw &w) { return Scales{{w.hd.x, w.hd.y, w.hd.z, w.hd.w}}; }
// Q3_K's 6-bit scales of half n (format/quant.rs:420-447, the kmask shuffle of the 12 bytes
// a0 | a1 | t): groups 0-3 and 4-7 of the half as bytes of two words
AH_DEV uint32_t q3_scw(const Scales &S, uint32_t n, uint32_t hi) {
    const uint32_t a = hi ? S.w[1] : S.w[0], t = S.w[2];
    return ((a >> (4 * n)) & 0x0F0F0F0Fu) | (((t >> (4 * n + 2 * hi)) & 0x03030303u) << 4);
}

// Side data of a super-block for the fold: d, dmin' and 16 f16 "min weights" per row, where the
// fold is acc += d P - dmin' (sum_k mw_k X_k) and X are the min-term operand's code sums:
//   Q4_K: dmin' = dmin, mw = m_j of the 8 sub-blocks (the operand's split sums, hi then lo);
//   Q2_K: dmin' = dmin, mw = m_g of the 16 groups (16-group sums);
//   Q3_K: dmin' = 4 d, mw = sc_g - 32 (the weight operand carries q + 4 = (q2 | h << 2), so the
//         -4 of each code returns as -4 d (sc_g - 32) X_g).
template <int TYPE>
AH_DEV void side(const Raw &w, const Scales &S, float &d, float &dm, uint32_t (&mw)[8]) {
    if constexpr (TYPE == AH_GGML_Q4_K) {
        d = ah_f16_bits_to_f32(w.hd.x & 0xffffu);
        dm = ah_f16_bits_to_f32(w.hd.x >> 16);
        const uint32_t s0 = S.w[1], s1 = S.w[2], s2 = S.w[3];
        const f16x2 m01 = {(_Float16)(float)q4k_scale<0, true>(s0, s1, s2), (_Float16)(float)q4k_scale<1, true>(s0, s1, s2)};
        const f16x2 m23 = {(_Float16)(float)q4k_scale<2, true>(s0, s1, s2), (_Float16)(float)q4k_scale<3, true>(s0, s1, s2)};
        const f16x2 m45 = {(_Float16)(float)q4k_scale<4, true>(s0, s1, s2), (_Float16)(float)q4k_scale<5, true>(s0, s1, s2)};
        const f16x2 m67 = {(_Float16)(float)q4k_scale<6, true>(s0, s1, s2), (_Float16)(float)q4k_scale<7, true>(s0, s1, s2)};
        mw[0] = mw[4] = as_u(m01);
        mw[1] = mw[5] = as_u(m23);
        mw[2] = mw[6] = as_u(m45);
        mw[3] = mw[7] = as_u(m67);
    } else if constexpr (TYPE == AH_GGML_Q2_K) {
        d = ah_f16_bits_to_f32(w.x.x & 0xffffu);
        dm = ah_f16_bits_to_f32(w.x.x >> 16);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t b = S.w[i >> 1] >> (16 * (i & 1));
            const f16x2 v = {(_Float16)(float)((b >> 4) & 15u), (_Float16)(float)((b >> 12) & 15u)};
            mw[i] = as_u(v);
        }
    } else {
        d = ah_f16_bits_to_f32(S.w[3] & 0xffffu);
        dm = 4.0f * d;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t sw = q3_scw(S, (uint32_t)(i >> 2), (uint32_t)((i >> 1) & 1));
            const uint32_t b = sw >> (16 * (i & 1));
            const f16x2 v = {(_Float16)(float)((int)(b & 0xffu) - 32), (_Float16)(float)((int)((b >> 8) & 0xffu) - 32)};
            mw[i] = as_u(v);
        }
    }
}

// The weight operand of the stage at position P, per K-step k (qs word k): the low run's four
// values (lo0, lo1) and the high run's (hi0, hi1), each exact in f16.  The scale operands
// (per run: multiplier and offset of nib4_times) are formed once per stage by `run_scales`.
struct RunScales {
    f16x2 ml, ol, mh, oh;
};
template <int TYPE, int P>
AH_DEV RunScales run_scales(const Scales &S, uint32_t h) {
    RunScales r;
    _Float16 sl, sh;  // the runs' group scales as multipliers of the byte values below
    _Float16 kl, kh;  // the byte values' place factors (the byte holds value * kl)
    if constexpr (TYPE == AH_GGML_Q4_K) {
        sl = (_Float16)(uint16_t)q4k_scale<2 * P, false>(S.w[1], S.w[2], S.w[3]);
        sh = (_Float16)(uint16_t)q4k_scale<2 * P + 1, false>(S.w[1], S.w[2], S.w[3]);
        kl = (_Float16)1.0f;
        kh = (_Float16)16.0f;
    } else if constexpr (TYPE == AH_GGML_Q2_K) {
        // groups 8n + 2 r0 + h and + 2: bytes h and h + 2 of scale word P (low nibbles)
        const uint32_t wd = S.w[P];
        sl = (_Float16)(float)((wd >> (8 * h)) & 15u);
        sh = (_Float16)(float)((wd >> (8 * h + 16)) & 15u);
        kl = (_Float16)(float)(1u << (4 * (P & 1)));      // pair r0 = 2 (P & 1) in place: 4^r0
        kh = (_Float16)(float)(1u << (4 * (P & 1) + 2));  // pair r0 + 1
    } else {
        const uint32_t sw = q3_scw(S, P >> 1, P & 1);  // groups 4 (P & 1) .. +3 of half P >> 1
        sl = (_Float16)(float)((int)((sw >> (8 * h)) & 0xffu) - 32);
        sh = (_Float16)(float)((int)((sw >> (8 * h + 16)) & 0xffu) - 32);
        kl = (_Float16)1.0f;
        kh = (_Float16)1.0f;
    }
    // (1024 + k v) * (s / k) - 1024 s / k = v s: s / k and 1024 s / k are exact in f16 (k a power
    // of two) and v s is representable, so the fused rounding is exact
    const _Float16 ml = sl / kl, mh = sh / kh;
    r.ml = (f16x2){ml, ml};
    r.mh = (f16x2){mh, mh};
    r.ol = (f16x2){ml * (_Float16)(-1024.0f), ml * (_Float16)(-1024.0f)};
    r.oh = (f16x2){mh * (_Float16)(-1024.0f), mh * (_Float16)(-1024.0f)};
    return r;
}
template <int TYPE, int P>
AH_DEV void convert_word(const Raw &w, const RunScales &rs, uint32_t k, uint32_t &lo0, uint32_t &lo1, uint32_t &hi0,
                         uint32_t &hi1) {
    const uint32_t qw = k == 0 ? w.q.x : k == 1 ? w.q.y : k == 2 ? w.q.z : w.q.w;
    uint32_t bl, bh;  // byte values (times their place factor) of the low and high run
    if constexpr (TYPE == AH_GGML_Q4_K) {
        bl = qw & 0x0F0F0F0Fu;
        bh = qw & 0xF0F0F0F0u;
    } else if constexpr (TYPE == AH_GGML_Q2_K) {
        constexpr uint32_t r0 = 2 * (P & 1);
        bl = qw & (0x03030303u << (2 * r0));
        bh = qw & (0x03030303u << (2 * r0 + 2));
    } else {
        constexpr uint32_t r0 = 2 * (P & 1), n = P >> 1;
        const uint32_t hw = k == 0 ? w.x.x : k == 1 ? w.x.y : k == 2 ? w.x.z : w.x.w;
        // v = q2 | hbit << 2 in 0..7 (the code plus 4), hbit = bit 4n + r of the hmask byte
        constexpr int sl = (int)(4 * n + r0) - 2, sh = sl + 1;
        const uint32_t hl = sl >= 0 ? hw >> sl : hw << -sl, hh = sh >= 0 ? hw >> sh : hw << -sh;
        bl = ((qw >> (2 * r0)) & 0x03030303u) | (hl & 0x04040404u);
        bh = ((qw >> (2 * r0 + 2)) & 0x03030303u) | (hh & 0x04040404u);
    }
    nib4_times(bl, rs.ml, rs.ol, lo0, lo1);
    nib4_times(bh, rs.mh, rs.oh, hi0, hi1);
}

}  // namespace dq

// Epilogue of the dequantize-once design: the wave's 2 x 2 tiles of 32 tokens x 32 rows.  As
// gemm_store: token scales applied (partials stay unscaled), lanes past n_out, tokens past n_tok
// and flagged tokens store out of range, output refusals recorded from a rare second pass over
// this lane's own stores, flagged tokens recomputed per row by the exact path.  `ts` is the
// wave's 64 token scales in LDS (staged at the start of the workgroup: two dependent global
// round trips here had cost ~4 us per tile).
template <int TYPE>
AH_DEV __attribute__((always_inline)) void dq_store(const GemmArgs &a, const GemmPartArgs &pa, const f32x16 (&acc)[2][2],
                                                    const float *ts, uint32_t row_w, uint32_t tok_w, uint32_t split,
                                                    uint32_t u_lo, uint32_t u_hi, const float *TS, uint32_t tok0,
                                                    uint8_t *win, uint32_t win_bytes) {
    const int lane = threadIdx.x & 63, j = lane & 31, h = lane >> 5;
    const uint32_t ntile = a.n_tok > tok_w ? (a.n_tok - tok_w < 64u ? a.n_tok - tok_w : 64u) : 0u;
    float *ybase = pa.splits == 1 ? pa.y + (size_t)tok_w * pa.n_out
                                  : pa.y + ((size_t)split * a.n_tok + tok_w) * pa.n_out;
    const __amdgpu_buffer_rsrc_t ry = ah_rsrc(ybase, ntile * pa.n_out * 4u);
    const bool scaled = pa.splits == 1;
    bool rl[2];
#pragma unroll
    for (int n = 0; n < 2; ++n) rl[n] = row_w + 32u * n + j < pa.n_out;
    // flagged tokens of the wave: lane l holds token l's scale
    const uint64_t fm = __builtin_amdgcn_ballot_w64(
        (uint32_t)lane < ntile && ah_ts_flagged(__builtin_bit_cast(uint32_t, ts[lane])));
    bool bad = false;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        // lanes of half h hold tokens 32m + 8q + 4h + i (q = r / 4, i = r % 4): four consecutive
        uint32_t sc[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(ts + 32 * m + 8 * q + 4 * h);
            sc[4 * q] = v.x;
            sc[4 * q + 1] = v.y;
            sc[4 * q + 2] = v.z;
            sc[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const uint32_t row = row_w + 32 * n + j;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t tl = 32 * m + 8 * (r / 4) + 4 * h + (r % 4);
                const bool ok = rl[n] && tl < ntile && !ah_ts_flagged(sc[r]);
                const float v = acc[m][n][r] * (scaled ? ah_ts_value(sc[r]) : 1.0f);
                bad = bad || (ok && !(__builtin_fabsf(v) < 0x1p31f));
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry,
                                                      ok ? (tl * pa.n_out + row) * 4u : kOob, 0, 0);
            }
        }
    }
    if (scaled && __builtin_amdgcn_ballot_w64(bad) != 0ull) {
        __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
        for (uint32_t e = 0; e < 64u; ++e) {
            const uint32_t m = e / 32, n = (e / 16) % 2, r = e % 16;
            const uint32_t tl = 32 * m + 8 * (r / 4) + 4 * h + (r % 4), row = row_w + 32 * n + j;
            if (!rl[n] || tl >= ntile || ah_ts_flagged(__builtin_bit_cast(uint32_t, ts[tl]))) continue;
            const float v = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ry, (tl * pa.n_out + row) * 4u, 0, 1));
            if (const uint32_t oc = ah_out_code(v)) ah_record(a.status, ah_out_key(pa.key0 + (uint64_t)(tok_w + tl) * pa.n_out + row, oc));
        }
    }
    // flagged tokens: the workgroup's, both token halves (`TS`: its 128 token scales), so that
    // the exact path's loop is the same in every wave
    (void)fm;
    const uint32_t nt = a.n_tok > tok0 ? (a.n_tok - tok0 < 128u ? a.n_tok - tok0 : 128u) : 0u;
    const uint64_t f0 = __builtin_amdgcn_ballot_w64((uint32_t)lane < nt && ah_ts_flagged(__builtin_bit_cast(uint32_t, TS[lane])));
    const uint64_t f1 =
        __builtin_amdgcn_ballot_w64(64u + (uint32_t)lane < nt && ah_ts_flagged(__builtin_bit_cast(uint32_t, TS[64 + lane])));
    if ((f0 | f1) != 0ull)
        exact_tokens<TYPE, 2>(a, pa, win, win_bytes, f0, f1, tok0, row_w, tok_w - tok0, tok_w - tok0 + ntile, ybase, scaled,
                              u_lo, u_hi);
}

// Epilogue of the prefill FFN's fused gate/up tiles (kFormTileFfn).  The wave's accumulators
// hold gate (n = 0) and up (n = 1) of the same 32 hidden indices for its 64 tokens.  They go
// through the wave's own 16 KB of LDS ([2][64 tokens][32 hidden] f32, token scales applied,
// flagged tokens replaced by the exact path's values), then each of 32 rounds takes two tokens,
// one per half-wave, 32 hidden values each: the optional f32 gate / up outputs, their output
// refusals, h = round_shift_32(silu_fixed(to_q32(gate)) * to_q32(up)) and quant_act of the
// 32-block, all in the reference FFN's refusal order (chart/ffn.rs:1712-1720, step/cols.rs:
// 1026-1067): the gate projection's outputs (key t * n_ff + k), the up projection's (past all
// gate keys), the elements' conversion or SwiGLU, then the hidden quantizer's blocks.
template <int TYPE>
AH_DEV __attribute__((always_inline)) void dq_ffn_store(const GemmArgs &a, const GemmPartArgs &pa,
                                                        const f32x16 (&acc)[2][2], const float *ts, float *E,
                                                        uint32_t hid_w, uint32_t tok_w) {
    const uint32_t lane = threadIdx.x & 63u, j = lane & 31u, h = lane >> 5;
    const uint32_t n_ff = pa.n_out, N = a.n_tok;
    const uint32_t ntile = N > tok_w ? (N - tok_w < 64u ? N - tok_w : 64u) : 0u;
    const uint32_t k = hid_w + j;
    const bool kl = k < n_ff;
    const uint64_t NF = (uint64_t)N * n_ff;
    const uint32_t nbh = (n_ff + 31) / 32, blk = hid_w / 32;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(ts + 32 * m + 8 * q + 4 * h);
            const uint32_t sc[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t tl = 32 * m + 8 * q + 4 * h + i;
                const float f = ah_ts_value(sc[i]);
                E[tl * 32 + j] = acc[m][0][4 * q + i] * f;
                E[2048 + tl * 32 + j] = acc[m][1][4 * q + i] * f;
            }
        }
    }
    // flagged tokens: both projections' rows by the exact path, the lane halves taking
    // alternate super-blocks
    uint64_t fm = __builtin_amdgcn_ballot_w64(lane < ntile && ah_ts_flagged(__builtin_bit_cast(uint32_t, ts[lane])));
    const uint32_t nb32 = (a.n_in + 31) / 32, nsb = a.kpad / 256;
    while (fm) {
        const uint32_t tl = (uint32_t)__builtin_ctzll(fm);
        fm &= fm - 1;
        const size_t t = (size_t)tok_w + tl;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const uint8_t *w = n ? a.ffn.w_up : pa.w;
            float v = kl ? exact_row<TYPE>(w + (size_t)k * pa.row_bytes, a.fcodes + t * a.n_in, a.fscales + t * nb32,
                                           a.n_in, 0u, nsb, h)
                         : 0.0f;
            v += __shfl_xor(v, 32, 64);
            if (h == 0) E[2048 * n + tl * 32 + j] = v;
        }
    }
    const size_t pitch = n_ff;
    for (uint32_t i = 0; i < 32u; ++i) {
        const uint32_t tl = 2 * i + h;
        const bool tv = tl < ntile, live = tv && kl;
        const uint64_t t = (uint64_t)tok_w + tl;
        const float g = E[tl * 32 + j], u = E[2048 + tl * 32 + j];
        const size_t e = (size_t)t * pitch + k;
        if (live) {
            if (a.ffn.gy) a.ffn.gy[e] = g;
            if (a.ffn.uy) a.ffn.uy[e] = u;
            if (const uint32_t oc = ah_out_code(g)) ah_record(a.status, ah_out_key(e, oc));
            if (const uint32_t oc = ah_out_code(u)) ah_record(a.status, ah_out_key(NF + e, oc));
        }
        const HiddenQ hq = swiglu_quant32(__builtin_bit_cast(uint32_t, g), __builtin_bit_cast(uint32_t, u), live);
        if (hq.err) ah_record(a.status, ah_out_key(2 * NF + e, (uint32_t)hq.err));
        if (live) a.ffn.h_codes[e] = (int8_t)hq.code;
        if (tv && j == 0) {
            const uint64_t bi = t * nbh + blk;
            if (hq.bad_block) ah_record(a.status, ah_out_key(3 * NF + bi, 7u));
            a.ffn.h_scales[bi] = (int64_t)hq.scale;
        }
    }
}

// A workgroup is 4 waves (2 x 2, each 64 rows x 64 tokens) over a 128 x 128 tile, two
// workgroups per CU.  The activation fragments come straight from global memory into registers
// (the operand in fragment order: one coalesced 1 KB load per fragment, a stage ahead, each
// fragment's registers reloaded for the next stage right after its MFMAs), so LDS only carries
// the converted weights: per stage 16 KB written and 32 KB of fragment reads, where staging the
// activations as well doubled that.  The raw weight bytes are requested two stages ahead; each
// stage converts the next stage's weights into the other plane while it multiplies (one word of
// each run per K-step, interleaved with the MFMAs), and one barrier per stage hands the plane over.
// At the end of a super-block the MFMA sums fold with the row's d, and the min term (Q4_K, Q2_K
// mins; Q3_K the codes' -4) rides on one more MFMA per tile.
//
// FFN (kFormTileFfn): the tile's 128 rows are 64 hidden indices of a gate/up pair: row
// 64 s + 32 n + i is hidden index 64 rtile + 32 s + i of the gate (n = 0) or up (n = 1)
// projection, so each wave's two row blocks are the gate and up of the same 32 hidden indices,
// and the epilogue (dq_ffn_store) writes the hidden QuantAct.  No split-K: the SwiGLU needs whole
// sums.  Its LDS grows to 64 KB (the epilogue's exchange reuses the planes), still two
// workgroups per CU.
template <int TYPE, bool FFN = false>
__global__ void __launch_bounds__(256, 2) gemm_dq_kernel(GemmArgs a) {
    static_assert(dq::served<TYPE>(), "dequantize-once design: Q4_K, Q2_K, Q3_K");
    constexpr uint32_t kSB = dq::sb_bytes<TYPE>();
    constexpr uint32_t kOD = 2 * dq::kPlane, kOM = kOD + 2048;
    constexpr uint32_t kOT = FFN ? 65536u : kOM + 8192;
    __shared__ __align__(16) uint8_t lds[kOT + 512];
    const uint32_t per = gridDim.x >> 3;
    const uint32_t L = (blockIdx.x & 7u) * per + (blockIdx.x >> 3);
    if (L >= a.n_wg) return;
    uint32_t pi = 0;
#pragma unroll
    for (uint32_t i = 1; i < kGemmMaxParts; ++i)
        if (i < a.n_parts && L >= a.p[i].wg_begin) pi = i;
    const GemmPartArgs &pa = a.p[pi];
    const uint32_t Lp = L - pa.wg_begin;
    const uint32_t tt = Lp % pa.tok_tiles, rest = Lp / pa.tok_tiles;
    const uint32_t split = rest % pa.splits, rtile = rest / pa.splits;

    const uint32_t tid = threadIdx.x, lane = tid & 63u, j = lane & 31u, h = lane >> 5;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wr = wv & 1u, wt = wv >> 1;  // the wave's row half and token half
    const uint32_t row0 = rtile * dq::kBM, tok0 = tt * dq::kBN;
    const uint32_t ntile = a.n_tok - tok0 < dq::kBN ? a.n_tok - tok0 : dq::kBN;
    // this thread's conversion row (32 per wave) and its byte offset; FFN: hidden index
    // 64 rtile + 32 (wv / 2) + j of the gate (even waves) or up (odd waves) projection
    const uint32_t crow = 32u * wv + j;
    const uint32_t csrc = FFN ? rtile * 64u + 32u * (wv >> 1) + j : row0 + crow;
    const bool clive = csrc < pa.n_out;
    const uint32_t croff = clive ? csrc * pa.row_bytes : 0u;
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(FFN && (wv & 1u) ? a.ffn.w_up : pa.w, pa.w_bytes);
    const uint32_t nkb = a.kpad / 16, nsb = a.kpad / 256;
    const uint32_t ntb = (a.n_tok + 31) / 32;
    // the wave's two 32-token blocks of the fragment-order operand
    const uint32_t tb0 = tok0 / 32 + 2 * wt;
    const __amdgpu_buffer_rsrc_t rf = ah_rsrc(a.xf, ntb * nkb * 1024u);
    const __amdgpu_buffer_rsrc_t rm = ah_rsrc(TYPE == AH_GGML_Q4_K ? a.xmin : a.xmin16, a.n_tok * nsb * 32u);

    const uint32_t nstages = a.kpad / kKS;
    const uint32_t st_begin = split * pa.stages_per_split;
    const uint32_t st_end = st_begin + pa.stages_per_split < nstages ? st_begin + pa.stages_per_split : nstages;

    uint8_t *const B[2] = {lds, lds + dq::kPlane};
    float *const Dd = reinterpret_cast<float *>(lds + kOD);  // [par][0..127] d, [par][128..255] dmin'
    uint8_t *const M = lds + kOM;                            // [par][128 rows][16] f16 min weights
    float *const TS = reinterpret_cast<float *>(lds + kOT);  // the tile's 128 token scales

    // activation fragment (token block tb0 + m, K-step k16 of stage st); past the split or the
    // operand: zeros (the rows of a partial token block past n_tok are never stored from)
    auto loadA = [&](uint32_t st, uint32_t m, uint32_t k16) -> f16x8 {
        const uint32_t off = (((tb0 + m) * nkb + st * 4 + k16) * 64 + lane) * 16u;
        return __builtin_bit_cast(f16x8, ah_ld128(rf, st < st_end ? off : kOob));
    };
    // the min-term operand of super-block sb for token tile m: lane (token j, half h) holds its
    // code sums 8h .. 8h + 7
    auto loadX = [&](uint32_t sb, uint32_t m) -> f16x8 {
        const uint32_t t = tok0 + 64u * wt + 32u * m + j;
        return __builtin_bit_cast(f16x8, ah_ld128(rm, t < a.n_tok ? (t * nsb + sb) * 32u + 16u * h : kOob));
    };

    f32x16 acc[2][2], P[2][2];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int n = 0; n < 2; ++n) acc[m][n] = P[m][n] = (f32x16){};
    dq::Scales S = {{0u, 0u, 0u, 0u}};  // scale words of the super-block being converted

    // a super-block's header at its first conversion: the scale words, and d, dmin' and the min
    // weights into parity `par` (both lane halves of a row write the same values)
    auto header = [&](const dq::Raw &w, uint32_t par) {
        S = dq::scales_of(w);
        float d, dm;
        uint32_t mw[8];
        dq::side<TYPE>(w, S, d, dm, mw);
        Dd[256 * par + crow] = d;
        Dd[256 * par + 128 + crow] = dm;
        *reinterpret_cast<u32x4 *>(M + par * 4096u + crow * 32u) = (u32x4){mw[0], mw[1], mw[2], mw[3]};
        *reinterpret_cast<u32x4 *>(M + par * 4096u + crow * 32u + 16u) = (u32x4){mw[4], mw[5], mw[6], mw[7]};
    };
    auto fetch = [&](auto pc, uint32_t st) -> dq::Raw {
        return dq::fetch<TYPE, decltype(pc)::value>(rs, croff + kSB * (st / 4), h, clive && st < st_end);
    };
    // the whole conversion of a stage (the prologue's; the loop interleaves it with the MFMAs)
    auto convert_all = [&](auto pc, const dq::Raw &w, uint8_t *plane) {
        constexpr int PC = decltype(pc)::value;
        const dq::RunScales r = dq::run_scales<TYPE, PC>(S, h);
#pragma unroll
        for (uint32_t k16 = 0; k16 < 4; ++k16) {
            uint32_t f0, f1, g0, g1;
            dq::convert_word<TYPE, PC>(w, r, k16, f0, f1, g0, g1);
            *reinterpret_cast<u32x2 *>(plane + dq::swz(crow, 2 * h + (k16 >> 1)) + 8 * (k16 & 1)) = (u32x2){f0, f1};
            *reinterpret_cast<u32x2 *>(plane + dq::swz(crow, 4 + 2 * h + (k16 >> 1)) + 8 * (k16 & 1)) = (u32x2){g0, g1};
        }
    };

    const uint32_t sw = (j >> 1) & 7u;
    auto fragB = [&](const uint8_t *buf, uint32_t n, uint32_t k16) -> f16x8 {
        const uint32_t r = 64u * wr + 32u * n + j;
        return *reinterpret_cast<const f16x8 *>(buf + r * 128u + 16u * ((2u * k16 + h) ^ sw));
    };

    // prologue: the token scales, stage 0's activation fragments, raw bytes of stages 0 and 1,
    // stage 0 converted
    f16x8 fa[4][2];
    if (wv == 0 && lane < 32u) {
        const u32x4 v = ah_ld128(ah_rsrc(a.tok_scale + tok0, ntile * 4u), 16u * lane);
        *reinterpret_cast<u32x4 *>(TS + 4 * lane) = v;
    }
#pragma unroll
    for (uint32_t k16 = 0; k16 < 4; ++k16)
#pragma unroll
        for (uint32_t m = 0; m < 2; ++m) fa[k16][m] = loadA(st_begin, m, k16);
    dq::Raw W[2];
    W[0] = fetch(std::integral_constant<int, 0>{}, st_begin);
    W[1] = fetch(std::integral_constant<int, 1>{}, st_begin + 1);
    header(W[0], 0u);
    convert_all(std::integral_constant<int, 0>{}, W[0], B[0]);
    ah_lds_barrier();

    f16x8 am[2];  // the min-term operand of the current super-block
    // Stage st at super-block position U (compile-time; slot U & 1), the super-block's side data
    // in parity `par`.
    auto stage = [&](auto uc, uint32_t st, uint32_t par) {
        constexpr int U = decltype(uc)::value, UN = (U + 1) & 3, PF = (U + 2) & 3;
        const uint8_t *Bc = B[U & 1];
        uint8_t *Bn = B[(U + 1) & 1];
        f16x8 fb[2][2];
        fb[0][0] = fragB(Bc, 0, 0);
        fb[0][1] = fragB(Bc, 1, 0);
        if constexpr (U == 0) {
            am[0] = loadX(st / 4, 0);
            am[1] = loadX(st / 4, 1);
        }
        W[U & 1] = fetch(std::integral_constant<int, PF>{}, st + 2);
        // the next stage's conversion (stage st + 1): scale operands, and its super-block header
        const dq::Raw &wn = W[(U + 1) & 1];
        if constexpr (UN == 0) header(wn, par ^ 1u);
        const dq::RunScales rsc = dq::run_scales<TYPE, UN>(S, h);
#pragma unroll
        for (uint32_t k16 = 0; k16 < 4; ++k16) {
            const uint32_t cb = k16 & 1u, nb = cb ^ 1u;
            if (k16 < 3) {
                fb[nb][0] = fragB(Bc, 0, k16 + 1);
                fb[nb][1] = fragB(Bc, 1, k16 + 1);
            }
            P[0][0] = mfma(fa[k16][0], fb[cb][0], P[0][0]);
            P[0][1] = mfma(fa[k16][0], fb[cb][1], P[0][1]);
            P[1][0] = mfma(fa[k16][1], fb[cb][0], P[1][0]);
            P[1][1] = mfma(fa[k16][1], fb[cb][1], P[1][1]);
            // this K-step's activation registers are free: the next stage's fragments
            fa[k16][0] = loadA(st + 1, 0, k16);
            fa[k16][1] = loadA(st + 1, 1, k16);
            uint32_t f0, f1, g0, g1;
            dq::convert_word<TYPE, UN>(wn, rsc, k16, f0, f1, g0, g1);
            *reinterpret_cast<u32x2 *>(Bn + dq::swz(crow, 2 * h + (k16 >> 1)) + 8 * (k16 & 1)) = (u32x2){f0, f1};
            *reinterpret_cast<u32x2 *>(Bn + dq::swz(crow, 4 + 2 * h + (k16 >> 1)) + 8 * (k16 & 1)) = (u32x2){g0, g1};
        }
        if constexpr (U == 3) {
            // fold the super-block: d * P - dmin' * (sum_k mw_k X_k), the latter one MFMA per tile
#pragma unroll
            for (uint32_t n = 0; n < 2; ++n) {
                const uint32_t r = 64u * wr + 32u * n + j;
                const float fd = Dd[256 * par + r], fdm = Dd[256 * par + 128 + r];
                const f16x8 bm = *reinterpret_cast<const f16x8 *>(M + par * 4096u + r * 32u + 16u * h);
#pragma unroll
                for (uint32_t m = 0; m < 2; ++m) {
                    const f32x16 pm = mfma(am[m], bm, (f32x16){});
                    // d P first, then dmin' pm (the same FMAs per element), while the MFMA completes
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[m][n][e] = __builtin_fmaf(fd, P[m][n][e], acc[m][n][e]);
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[m][n][e] = __builtin_fmaf(-fdm, pm[e], acc[m][n][e]);
                    P[m][n] = (f32x16){};
                }
            }
        }
        // the next stage's weights are in LDS and every wave is done with this stage's plane
        ah_lds_barrier();
    };
    uint32_t par = 0;
    for (uint32_t st = st_begin; st < st_end; st += 4) {
        stage(std::integral_constant<int, 0>{}, st, par);
        stage(std::integral_constant<int, 1>{}, st + 1, par);
        stage(std::integral_constant<int, 2>{}, st + 2, par);
        stage(std::integral_constant<int, 3>{}, st + 3, par);
        par ^= 1u;
    }
    if constexpr (FFN) {
        dq_ffn_store<TYPE>(a, pa, acc, TS + 64u * wt, reinterpret_cast<float *>(lds) + 4096u * wv,
                           rtile * 64u + 32u * wr, tok0 + 64u * wt);
    } else {
        static_assert(kOT >= xp::kWinBytes + 4 * xp::kBatch * 2 * 256u,
                      "the exact path stages a token window and its sums in the planes");
        dq_store<TYPE>(a, pa, acc, TS + 64u * wt, row0 + 64u * wr, tok0 + 64u * wt, split, st_begin / 4, st_end / 4, TS,
                       tok0, lds, kOT);
    }
}

}  // namespace

namespace {

// Stages of 64 the kernel for `type` runs over K, its unroll, and its workgroup tile.
struct GemmGeom {
    uint32_t nstages, unroll, rows, toks;
};
GemmGeom geom_of(uint32_t type, uint32_t n_in, uint32_t kpad, uint32_t waves = 4, uint32_t kind = kGemmKindRb) {
    const uint32_t rows = 32u * rb::kNN * waves;
    // int8: stages of 4 blocks (Q4_K: half super-blocks, split in whole super-blocks)
    if (kind == kGemmKindI8) return {i8::stages(n_in), type == AH_GGML_Q4_K ? 2u : 1u, rows, i8::kTok};
    if (kind == kGemmKindTile) return {kpad / kKS, 4, dq::kBM, dq::kBN};
    if (ah_blk32((int)type)) return {(n_in + 2 * kKS - 1) / (2 * kKS) * 2, 2, rows, rb::tok_of(type)};
    return {kpad / kKS, 4, rows, rb::tok_of(type)};  // K-quants: whole super-blocks
}

// Stages per split for a requested split count: a multiple of the unroll.
uint32_t per_split(const GemmGeom &g, uint32_t splits) {
    uint32_t per = (g.nstages + splits - 1) / splits;
    return (per + g.unroll - 1) / g.unroll * g.unroll;
}

}  // namespace

// Split-K count for an n_tok x n_out GEMM on `cus` compute units.  Cost model (microseconds),
// fitted to a sweep of every valid split count over the configs[3] and configs[4] prefill shapes
// at N = 512 on MI355X (it picks the measured best for all 13):
//   the busiest CU runs ceil(workgroups / cus) workgroups of `per` stages, c_type us a stage
//   (a second resident Q4_K workgroup shares the CU's throughput rather than adding to it);
//   a split GEMM adds the reduction: 4.8 us fixed plus the partials' write and read-back,
//   (splits + 1) * n_tok * n_out * 4 bytes at 0.253 us per MB.
uint32_t ah_gemm_pick_splits(uint32_t type, uint32_t n_out, uint32_t n_in, uint32_t n_tok,
                             uint32_t cus, uint32_t kind) {
    const bool int8 = kind == kGemmKindI8;
    const GemmGeom g = geom_of(type, n_in, (n_in + 255) / 256 * 256, 4, kind);
    const uint64_t tiles = (uint64_t)((n_out + g.rows - 1) / g.rows) * ((n_tok + g.toks - 1) / g.toks);
    const double c = kind == kGemmKindTile ? 0.55 : int8 ? 1.0 : ah_blk32((int)type) ? 0.806 : type == AH_GGML_Q4_K ? 0.400 : 1.081;
    uint32_t best = 1;
    double best_cost = 1e30;
    for (uint32_t want = 1; want <= 64 && want <= g.nstages; ++want) {
        const uint32_t per = per_split(g, want);
        const uint32_t used = (g.nstages + per - 1) / per;
        if (used != want) continue;
        const double waves = (double)((tiles * used + cus - 1) / cus);
        double cost = waves * per * c;
        if (used > 1) cost += 4.8 + (double)(used + 1) * n_tok * n_out * 4.0 * 0.253e-6;
        if (cost < best_cost) {
            best_cost = cost;
            best = used;
        }
    }
    return best;
}

// Parts one GEMM launch of `type` may hold.
uint32_t ah_gemm_max_parts(uint32_t type) { return rb::max_parts_of(type); }

// 4-wave workgroups (tiles x splits) of one part.
uint32_t ah_gemm_part_wg4(uint32_t type, uint32_t n_out, uint32_t n_in, uint32_t n_tok, uint32_t splits,
                          uint32_t kind) {
    const GemmGeom g = geom_of(type, n_in, (n_in + 255) / 256 * 256, 4, kind);
    return ((n_out + g.rows - 1) / g.rows) * ((n_tok + g.toks - 1) / g.toks) * splits;
}

// Workgroup form for a launch whose parts take n_wg4 workgroups on 4-wave tiles (Q8_0 and Q6_K;
// Q4_K's 64-token tiles already put two workgroups on a CU):
//   kForm4x4: 4 waves, 4-slot ring (64 KB), when the 4-wave grid is past two workgroups per CU;
//   kForm2x2: 2 waves, 2-slot ring (32 KB, four per CU), when it holds more workgroups than CUs
//             but at most two per CU -- a few CUs would run a second round after the rest;
//   kForm2x4: 2 waves, 4-slot ring, when it fits one workgroup per CU -- the same busy SIMDs
//             spread over every CU, halving each CU's load on its texture unit and LDS.
// Measured at N = 512 (A/B in one run): 8960x1536 Q8_0 48.8 -> 43.3 us, Q6_K 54.4 -> 47.7 on
// kForm2x2; 4864x896 23.5 -> 22.6, 1536x8960 46.6 -> 45.7 (Q6_K 55.3 -> 51.8) on kForm2x4.
uint32_t ah_gemm_pick_waves(uint32_t type, uint64_t n_wg4, uint32_t cus, bool int8) {
    if (int8) return n_wg4 <= cus ? kFormI8x2 : kFormI8x4;
    if (type == AH_GGML_Q4_K) return kForm4x4;
    return n_wg4 <= cus ? kForm2x4 : n_wg4 <= 2ull * cus ? kForm2x2 : kForm4x4;
}

// ---- MFMA peak probe ---------------------------------------------------------------------------
//
// The instruction's own ceiling, measured rather than quoted: a loop with no memory traffic that
// issues nothing but the MFMA (KIND 0: v_mfma_i32_32x32x32_i8, KIND 1: v_mfma_f32_32x32x16_f16)
// into 8 independent accumulators whose operands come from memory (so nothing is a compile-time
// constant) and differ per accumulator; every accumulator is folded into a per-thread sink, so
// no MFMA can be dropped (the emitted loop is 8 back-to-back MFMAs and a counter).  Each
// iteration depends on the last through its accumulator.
namespace {
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
constexpr int kProbeAcc = 8;

template <int KIND>
__global__ void __launch_bounds__(256) mfma_probe_kernel(const uint32_t *__restrict__ seed, uint32_t iters,
                                                         uint32_t *__restrict__ sink) {
    const uint32_t t = threadIdx.x & 63;
    uint32_t acc_x = 0;
    if constexpr (KIND == 0) {
        v4i a[kProbeAcc], b;
#pragma unroll
        for (int i = 0; i < kProbeAcc; ++i)
            a[i] = (v4i){(int)(seed[0] ^ t ^ i), (int)seed[1], (int)(seed[2] + i), (int)seed[3]};
        b = (v4i){(int)seed[4], (int)(seed[5] ^ t), (int)seed[6], (int)seed[7]};
        v16i c[kProbeAcc];
#pragma unroll
        for (int i = 0; i < kProbeAcc; ++i) c[i] = (v16i){};
        for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
            for (int i = 0; i < kProbeAcc; ++i) c[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b, c[i], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < kProbeAcc; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc_x ^= (uint32_t)c[i][r];
    } else {
        f16x8 a[kProbeAcc], b;
#pragma unroll
        for (int i = 0; i < kProbeAcc; ++i) {
            const u32x4 v = {seed[0] ^ t, seed[1] + (uint32_t)i, seed[2], seed[3]};
            a[i] = __builtin_bit_cast(f16x8, v & (u32x4){0x3bff3bffu, 0x3bff3bffu, 0x3bff3bffu, 0x3bff3bffu});
        }
        const u32x4 vb = {seed[4], seed[5] ^ t, seed[6], seed[7]};
        b = __builtin_bit_cast(f16x8, vb & (u32x4){0x3bff3bffu, 0x3bff3bffu, 0x3bff3bffu, 0x3bff3bffu});
        f32x16 c[kProbeAcc];
#pragma unroll
        for (int i = 0; i < kProbeAcc; ++i) c[i] = (f32x16){};
        for (uint32_t it = 0; it < iters; ++it) {
#pragma unroll
            for (int i = 0; i < kProbeAcc; ++i) c[i] = mfma(a[i], b, c[i]);
        }
        float fsum = 0.0f;  // a float sum: this compiler folded an XOR of the bit patterns to zero
#pragma unroll
        for (int i = 0; i < kProbeAcc; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) fsum += c[i][r];
        acc_x = __builtin_bit_cast(uint32_t, fsum);
    }
    sink[blockIdx.x * blockDim.x + threadIdx.x] = acc_x;
}
}  // namespace

// Runs the probe on `stream` (two 256-thread workgroups per CU: 2 waves per SIMD, which the 128
// accumulator registers of each wave allow) and returns the rate in tera-ops per second (int8:
// 2*32*32*32 ops per MFMA; f16: 2*32*32*16 flops), timed with HIP events.
hipError_t ah_probe_mfma(uint32_t kind, uint32_t cus, const uint32_t *d_seed, uint32_t *d_sink,
                         hipStream_t stream, double *tops) {
    const uint32_t grid = 2 * cus, iters = 8192;
    hipEvent_t e0, e1;
    hipError_t e = hipEventCreate(&e0);
    if (e != hipSuccess) return e;
    e = hipEventCreate(&e1);
    if (e != hipSuccess) {
        (void)hipEventDestroy(e0);
        return e;
    }
    float ms = 0.0f;
    for (int rep = 0; rep < 2 && e == hipSuccess; ++rep) {  // the first run warms up the clocks
        e = hipEventRecord(e0, stream);
        if (e != hipSuccess) break;
        if (kind == 0) hipLaunchKernelGGL(mfma_probe_kernel<0>, dim3(grid), dim3(256), 0, stream, d_seed, iters, d_sink);
        else hipLaunchKernelGGL(mfma_probe_kernel<1>, dim3(grid), dim3(256), 0, stream, d_seed, iters, d_sink);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipEventRecord(e1, stream);
        if (e == hipSuccess) e = hipEventSynchronize(e1);
        if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (e != hipSuccess) return e;
    const double per = kind == 0 ? 2.0 * 32 * 32 * 32 : 2.0 * 32 * 32 * 16;
    const double ops = per * kProbeAcc * iters * ((double)grid * 4);  // 4 waves per workgroup
    *tops = ms > 0.0f ? ops / (ms * 1e-3) / 1e12 : 0.0;
    return hipSuccess;
}

hipError_t ah_launch_gemm(uint32_t type, uint32_t n_parts, const GemmPartDesc *parts, uint32_t n_in,
                          uint32_t n_tok, uint32_t kpad, const _Float16 *xh, const _Float16 *xf, const _Float16 *xmin,
                          const _Float16 *xmin16,
                          const float *tok_scale, const int8_t *fcodes, const int64_t *fscales,
                          const int8_t *xc, const uint32_t *xsp, const uint32_t *xsx,
                          unsigned long long *status, uint32_t form, hipStream_t stream, const GemmFfn *ffn) {
    const bool mixed = type == kGemmMixedKQuant;  // Q4_K and Q6_K parts, 4-wave form
    const bool int8 = form == kFormI8x4 || form == kFormI8x2;
    const bool ffn_form = form == kFormTileFfn;
    const bool tile = form == kFormTile || ffn_form;
    if (n_parts == 0 || n_parts > (mixed || tile ? kGemmMaxParts : rb::max_parts_of(type))) return hipErrorInvalidValue;
    if (ffn_form && (!ffn || !ffn->w_up || !ffn->h_codes || !ffn->h_scales || n_parts != 1 || parts[0].splits > 1))
        return hipErrorInvalidValue;
    if (int8 && ((type != AH_GGML_Q8_0 && type != AH_GGML_Q4_K) || !xc || !xsp || (type == AH_GGML_Q4_K && !xsx) ||
                 n_parts != 1))
        return hipErrorInvalidValue;
    if (tile && (!xf || (type != AH_GGML_Q4_K && type != AH_GGML_Q2_K && type != AH_GGML_Q3_K) ||
                 (type != AH_GGML_Q4_K && !xmin16)))
        return hipErrorInvalidValue;
    if (!int8 && !tile && (mixed || type == AH_GGML_Q4_K || form > kForm2x4)) form = kForm4x4;
    const uint32_t kind = int8 ? kGemmKindI8 : tile ? kGemmKindTile : kGemmKindRb;
    const uint32_t waves = form == kForm4x4 || form == kFormI8x4 || tile ? 4u : 2u;
    GemmArgs a;
    a.n_parts = n_parts;
    a.n_in = n_in;
    a.n_tok = n_tok;
    a.kpad = kpad;
    a.xh = xh;
    a.xf = xf;
    a.xmin = xmin;
    a.xmin16 = xmin16;
    a.tok_scale = tok_scale;
    a.fcodes = fcodes;
    a.status = status;
    a.fscales = fscales;
    a.xc = xc;
    a.xsp = xsp;
    a.xsx = xsx;
    a.ffn = ffn_form ? *ffn : GemmFfn{};
    uint32_t wg = 0;
    for (uint32_t i = 0; i < kGemmMaxParts; ++i) {
        GemmPartArgs &P = a.p[i];
        if (i >= n_parts) {
            P = a.p[0];
            P.wg_begin = 0xFFFFFFFFu;
            continue;
        }
        const GemmPartDesc &d = parts[i];
        const uint32_t pt = mixed ? d.type : type;
        if (mixed && pt != AH_GGML_Q4_K && pt != AH_GGML_Q6_K) return hipErrorInvalidValue;
        const GemmGeom g = geom_of(pt, n_in, kpad, waves, kind);
        const uint32_t per = per_split(g, d.splits ? d.splits : 1);
        P.w = d.w;
        P.w_bytes = d.w_bytes;
        P.row_bytes = d.row_bytes;
        P.n_out = d.n_out;
        P.stages_per_split = per;
        P.splits = (g.nstages + per - 1) / per;
        if (P.splits != (d.splits ? d.splits : 1)) return hipErrorInvalidValue;  // planned with per_split
        P.y = P.splits == 1 ? d.y : d.partials;
        P.wg_begin = wg;
        P.tok_tiles = (n_tok + g.toks - 1) / g.toks;
        P.type = pt;
        P.key0 = d.key0;
        const uint32_t rows = ffn_form ? g.rows / 2 : g.rows;  // FFN: a tile's rows are hidden pairs
        wg += ((d.n_out + rows - 1) / rows) * P.tok_tiles * P.splits;
    }
    a.n_wg = wg;
    if (wg == 0) return hipSuccess;
    const dim3 rb_grid((a.n_wg + 7) / 8 * 8);
    const dim3 blk(64 * waves);
#define AH_GFORMS(T)                                                                                    \
    if (form == kForm2x2) hipLaunchKernelGGL((gemm_rb_kernel<T, 2, 2>), rb_grid, blk, 0, stream, a);    \
    else if (form == kForm2x4) hipLaunchKernelGGL((gemm_rb_kernel<T, 2, 4>), rb_grid, blk, 0, stream, a); \
    else hipLaunchKernelGGL((gemm_rb_kernel<T, 4, 4>), rb_grid, blk, 0, stream, a);
    if (ffn_form) {
        if (type == AH_GGML_Q4_K) hipLaunchKernelGGL((gemm_dq_kernel<AH_GGML_Q4_K, true>), rb_grid, dim3(256), 0, stream, a);
        else if (type == AH_GGML_Q2_K) hipLaunchKernelGGL((gemm_dq_kernel<AH_GGML_Q2_K, true>), rb_grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL((gemm_dq_kernel<AH_GGML_Q3_K, true>), rb_grid, dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    if (tile) {
        if (type == AH_GGML_Q4_K) hipLaunchKernelGGL(gemm_dq_kernel<AH_GGML_Q4_K>, rb_grid, dim3(256), 0, stream, a);
        else if (type == AH_GGML_Q2_K) hipLaunchKernelGGL(gemm_dq_kernel<AH_GGML_Q2_K>, rb_grid, dim3(256), 0, stream, a);
        else hipLaunchKernelGGL(gemm_dq_kernel<AH_GGML_Q3_K>, rb_grid, dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    if (form == kFormI8x4) {
        if (type == AH_GGML_Q4_K) hipLaunchKernelGGL((gemm_i8_kernel<AH_GGML_Q4_K, 4>), rb_grid, blk, 0, stream, a);
        else hipLaunchKernelGGL((gemm_i8_kernel<AH_GGML_Q8_0, 4>), rb_grid, blk, 0, stream, a);
        return hipGetLastError();
    }
    if (form == kFormI8x2) {
        if (type == AH_GGML_Q4_K) hipLaunchKernelGGL((gemm_i8_kernel<AH_GGML_Q4_K, 2>), rb_grid, blk, 0, stream, a);
        else hipLaunchKernelGGL((gemm_i8_kernel<AH_GGML_Q8_0, 2>), rb_grid, blk, 0, stream, a);
        return hipGetLastError();
    }
    switch (type) {
    case kGemmMixedKQuant: hipLaunchKernelGGL(gemm_rb_kquant_kernel, rb_grid, blk, 0, stream, a); break;
    case AH_GGML_Q8_0: AH_GFORMS(AH_GGML_Q8_0) break;
    case AH_GGML_Q5_0: AH_GFORMS(AH_GGML_Q5_0) break;
    case AH_GGML_Q4_K: hipLaunchKernelGGL((gemm_rb_kernel<AH_GGML_Q4_K, 4, 4>), rb_grid, blk, 0, stream, a); break;
    case AH_GGML_Q6_K: AH_GFORMS(AH_GGML_Q6_K) break;
    default: return hipErrorInvalidValue;
    }
#undef AH_GFORMS
    return hipGetLastError();
}

// One reduction launch for every part with splits > 1 (kReduceMaxParts per launch).
hipError_t ah_launch_splitk_reduce(uint32_t n_parts, const GemmPartDesc *parts, uint32_t n_tok,
                                   const float *tok_scale, unsigned long long *status, hipStream_t stream) {
    uint32_t i = 0;
    while (i < n_parts) {
        ReduceArgs r;
        r.tok_scale = tok_scale;
        r.status = status;
        r.n_tok = n_tok;
        r.n_parts = 0;
        bool vec = true;
        for (; i < n_parts && r.n_parts < kReduceMaxParts; ++i) {
            const GemmPartDesc &d = parts[i];
            if (d.splits <= 1 || d.n_out == 0) continue;
            const size_t n = (size_t)n_tok * d.n_out;
            vec = vec && n % 4 == 0 && (reinterpret_cast<uintptr_t>(d.partials) & 15u) == 0 &&
                  (reinterpret_cast<uintptr_t>(d.y) & 15u) == 0;
            ReducePart &P = r.p[r.n_parts++];
            P.part = d.partials;
            P.y = d.y;
            P.n_out = d.n_out;
            P.splits = d.splits;
            P.key0 = d.key0;
        }
        if (r.n_parts == 0) continue;
        uint64_t total = 0;
        for (uint32_t k = 0; k < r.n_parts; ++k) {
            r.p[k].begin = total;
            const uint64_t n = (uint64_t)n_tok * r.p[k].n_out;
            total += vec ? n / 4 : n;
        }
        for (uint32_t k = r.n_parts; k < kReduceMaxParts; ++k) {
            r.p[k] = r.p[0];
            r.p[k].begin = ~0ull;
        }
        r.total = total;
        uint64_t rg = (total + 255) / 256;
        if (rg > 8192) rg = 8192;
        if (vec) hipLaunchKernelGGL(splitk_reduce<true>, dim3((uint32_t)rg), dim3(256), 0, stream, r);
        else hipLaunchKernelGGL(splitk_reduce<false>, dim3((uint32_t)rg), dim3(256), 0, stream, r);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
