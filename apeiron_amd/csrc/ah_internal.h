// ah_internal.h -- shared device helpers and kernel argument blocks of the gfx950 backend.
//
// The arithmetic restated here follows the reference contract:
//   to_q32            num/fp.rs:186-230 (round half away from zero, exact on the f32 fields)
//   act_scale         kern/pow2.rs:11-39 (least power of two S with 127*S >= absmax)
//   quant_act codes   chart/mod.rs:258-334 (q + [2r >= S], sign applied, |code| <= 127)
//   dequantizes       chart/mod.rs:105-134 (every S*code must fit int64)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "apeiron_hip.h"

#define AH_DEV __device__ __forceinline__

// Types of 32-element blocks with one f16 scale each (Q8_0, Q5_0): one group per block, the same
// unit, stage and split geometry in every kernel.
constexpr bool ah_blk32(int t) { return t == AH_GGML_Q8_0 || t == AH_GGML_Q5_0; }
// K-quant families with no GEMM form of their own (their prefill is one GEMV launch per token).
constexpr bool ah_k23(int t) { return t == AH_GGML_Q2_K || t == AH_GGML_Q3_K; }

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Status word: the earliest failing element wins (atomicMin over (index << 8) | code).  Input
// conversion failures are ordered before quantizer failures, as the boundary converts the whole
// f32 vector before quant_act runs.
#define AH_ST_NONE 0xFFFFFFFFFFFFFFFFull
#define AH_QUANT_ORDER_BASE (1ull << 48)
// Output refusals come after every input refusal of the call (the reference converts and
// quantizes before it projects) and are ordered by output index (token-major for the GEMM, as
// matmat_q8act reports its first failing column).
#define AH_OUTPUT_ORDER_BASE (1ull << 56)

AH_DEV void ah_record(unsigned long long *st, unsigned long long key) {
    if (st) atomicMin(st, key);
}

// The refusal the exact contract makes for an output of real value y (ops/matvec.rs:35-37,
// 113-115): the i128 sum of Q32.32 products is y * 2^64, so |y| >= 2^63 leaves i128
// (AccumulatorOverflow, 8); round_shift_32 of it is y * 2^32, so |y| >= 2^31 leaves i64
// (OutputOverflow, 9).  A NaN (an f32 fold that overflowed both ways) counts as the former.
// Values within the f32 fold's tolerance of either bound may be classed either way.
AH_DEV uint32_t ah_out_code(float y) {
    const float a = __builtin_fabsf(y);
    return !(a < 0x1p63f) ? 8u : a >= 0x1p31f ? 9u : 0u;
}
AH_DEV unsigned long long ah_out_key(uint64_t index, uint32_t code) {
    const uint64_t i = index < (1ull << 47) ? index : (1ull << 47) - 1;
    return AH_OUTPUT_ORDER_BASE + (i << 8) + code;
}

// ---- buffer resources: range-checked loads (out-of-range lanes read 0, never fault) ----

AH_DEV __amdgpu_buffer_rsrc_t ah_rsrc(const void *p, uint32_t bytes) {
    // The range check drops a whole dword that straddles the end, and GGUF payloads are only
    // 2-byte multiples (34-, 210-byte blocks), so the range is rounded up to whole dwords.  The
    // extra 0-3 bytes share an aligned dword with payload bytes, so they can never touch a page
    // the payload does not.  word3 0x00020000: the gfx9-family raw buffer format.
    const uint32_t rounded = bytes > 0xFFFFFFFCu ? 0xFFFFFFFCu : (bytes + 3u) & ~3u;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)rounded,
                                             0x00020000);
}
AH_DEV u32x4 ah_ld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}
// Streamed weight bytes: read once per launch, so the load carries the non-temporal hint (nt),
// which keeps them from displacing cached lines and measurably raises the streaming rate.
AH_DEV u32x4 ah_ld128_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 2));
}
AH_DEV uint32_t ah_ld32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

// Workgroup barrier for LDS traffic only: this wave's LDS operations are complete before it
// arrives, and global loads stay in flight (__syncthreads also waits for every outstanding global
// load, which would drain a prefetch).  The memory clobber keeps the compiler from moving memory
// operations across it.
AH_DEV void ah_lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// The same after this wave's vector memory loads have come down to at most N outstanding (they
// complete in issue order), for direct-to-LDS loads that the compiler does not wait for.
template <int N> AH_DEV void ah_vm_lds_barrier() {
    static_assert(N >= 0 && N <= 63, "vmcnt is a 6-bit count");
    __asm__ volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// ---- exact integer helpers ----

AH_DEV int32_t ah_sdot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
// A dot chain's first step: the three-operand form with an inline 0 accumulator.  From the
// builtin the compiler picks the accumulating two-operand v_dot4c, which first moves 0 into its
// destination: one VALU instruction per chain.
AH_DEV int32_t ah_sdot4_first(uint32_t a, uint32_t b) {
    int32_t d;
    __asm__("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
AH_DEV uint32_t ah_alignbyte(uint32_t hi, uint32_t lo, uint32_t sh) {
    return __builtin_amdgcn_alignbyte(hi, lo, sh);
}
AH_DEV float ah_f16_bits_to_f32(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;  // exact (v_cvt_f32_f16 keeps subnormals)
}

// f32 bits -> |round_half_away(v * 2^32)| and sign; returns 0, 10 (non-finite) or 11 (range).
AH_DEV int ah_to_q32_mag(uint32_t bits, uint64_t &mag, bool &neg) {
    uint32_t e = (bits >> 23) & 0xffu;
    neg = (bits >> 31) != 0;
    if (e == 0xffu) return 10;
    uint32_t frac = bits & 0x7fffffu;
    uint64_t m = e ? (uint64_t)(frac | 0x800000u) : (uint64_t)frac;
    uint32_t ee = e ? e : 1u;
    if (ee >= 118u) {
        uint32_t k = ee - 118u;
        if (k > 40u) return 11;
        mag = m << k;  // m < 2^24, k <= 40: below 2^64
    } else {
        uint32_t sh = 118u - ee;
        mag = sh > 24u ? 0ull : ((m + (1ull << (sh - 1u))) >> sh);
    }
    const uint64_t lim = 1ull << 63;
    if (neg ? mag > lim : mag >= lim) return 11;
    return 0;
}

// Exponent of the activation scale: -1 for absmax == 0 (S = 0), 63 for act_scale's None,
// else e with S = 2^e the least power of two such that 127*S >= absmax.
// With b = bit length of absmax and e0 = max(0, b - 7): 127 * 2^(e0 - 1) < 2^(b-1) <= absmax,
// so the least e is e0 when 127 * 2^e0 >= absmax and e0 + 1 otherwise (127 * 2^(e0+1) >= 2^b).
AH_DEV int ah_act_scale_exp(uint64_t absmax) {
    if (absmax == 0) return -1;
    const int b = 64 - __builtin_clzll(absmax);
    const int e0 = b > 7 ? b - 7 : 0;
    const int e = e0 + (absmax > (127ull << e0) ? 1 : 0);
    return e > 62 ? 63 : e;
}

// The quant_act code of one magnitude under S = 2^e (e >= 0): q + [2r >= S] with the sign.
// Sets `bad` when S*code leaves int64 (QuantAct::dequantizes).
AH_DEV int ah_act_code(uint64_t mag, bool neg, int e, bool &bad) {
    uint64_t c = e == 0 ? mag : (mag >> e) + ((mag >> (e - 1)) & 1ull);
    // c <= 127 by the choice of S.  The product c*2^e must fit: positive < 2^63, negative <= 2^63.
    if (e >= 56) {
        uint64_t lim = 1ull << (63 - e);
        if (neg ? c > lim : c >= lim) bad = true;
    }
    return neg ? -(int)c : (int)c;
}

// The quant_act code of an f32 element under S = 2^e (0 <= e <= 62) in 32-bit arithmetic, equal
// to ah_act_code(ah_to_q32_mag(bits), e).  With |x| = m * 2^(ee - 150) (m the 24-bit significand,
// ee >= 1 the biased exponent, subnormals taking ee = 1), |x| * 2^32 = m * 2^(ee - 118).
// rhu(v, k) = ((v >> (k - 1)) + 1) >> 1 rounds v / 2^k half up (k >= 1), which is to_q32's and
// the code's rounding on magnitudes.  For ee >= 118, to_q32 is exact and the code is one rounding
// of m by sh = e + 118 - ee (sh >= 17 in any block whose scale is 2^e: m >= 2^23, code <= 127);
// for ee < 118, to_q32 rounds m by 2^(118 - ee) first and the code rounds that by 2^e.  Shift
// counts are clamped at 25: m < 2^24 makes every larger shift give the same 0.
AH_DEV int ah_act_code_f32(uint32_t bits, int e, bool &bad) {
    const uint32_t eb = (bits >> 23) & 0xffu;
    const uint32_t ee = eb ? eb : 1u;
    const uint32_t m = (bits & 0x7fffffu) | (eb ? 0x800000u : 0u);
    // Both cases are evaluated (shift counts clamped to [0, 25]) and one is selected, so a wave
    // whose lanes straddle ee = 118 does not run two branches.
    const int sh = e + 118 - (int)ee;
    const uint32_t ka = sh < 1 ? 0u : (sh - 1 > 25 ? 25u : (uint32_t)(sh - 1));
    const uint32_t ca = ((m >> ka) + 1u) >> 1;
    const int d1 = 117 - (int)ee;
    const uint32_t k1 = d1 < 0 ? 0u : (d1 > 25 ? 25u : (uint32_t)d1);
    const uint32_t mag = ((m >> k1) + 1u) >> 1;
    const uint32_t kb = e < 1 ? 0u : (e - 1 > 25 ? 25u : (uint32_t)(e - 1));
    const uint32_t cb = e == 0 ? mag : ((mag >> kb) + 1u) >> 1;
    const uint32_t c = ee >= 118u ? ca : cb;
    const bool neg = (bits >> 31) != 0;
    if (e >= 56) {
        const uint32_t lim = 1u << (63 - e);
        if (neg ? c > lim : c >= lim) bad = true;
    }
    return neg ? -(int)c : (int)c;
}

// ---- kernel argument blocks ----

enum { AH_SRC_F32 = 0, AH_SRC_Q32 = 1, AH_SRC_CODES = 2 };

struct GemvPart {
    const uint8_t *w;      // GGUF payload (device)
    uint64_t w_bytes;      // n_out * row_bytes
    const void *x;         // f32 / int64 activation, or int8 codes
    const int64_t *scales; // with AH_SRC_CODES
    float *y;
    int32_t *dots;         // optional exact group dots [n_out][ngroups]
    uint32_t n_out, n_in, row_bytes;
    uint32_t units;        // work units per row (Q8_0 blocks, K-quant super-blocks)
    uint32_t rows_per_tile;// whole rows per tile (per workgroup tile or per wave tile)
    uint32_t lanes;        // wave-tile kernel: lanes per row (a power of two <= 64)
    uint32_t wg_begin;     // first workgroup of this part in a grouped launch
    uint32_t wg_count;     // workgroups of this part
    uint32_t src;          // AH_SRC_*
    uint32_t type;         // GGUF type (AH_GGML_*): read by the mixed-type streaming plan
    uint32_t key_tok;      // token (column) index of a prefill served by GEMV launches: input
                           // refusals are keyed key_tok * n_in + element; 0 otherwise
    uint64_t out_key0;     // added to the output refusal key (row): the part's and the token's place
                           // in a grouped prefill, token-major per part as matmat_q8act reports
};

// The parts of a streaming launch without a workgroup table: a single projection, or a plan of at
// most kStreamArgParts parts (whole workgroups per part, p[i].wg_begin / wg_count), passed in the
// kernel arguments so that a workgroup reaches its part, its weights and its activation without a
// dependent descriptor load.
constexpr uint32_t kStreamArgParts = 4;
struct StreamParts {
    GemvPart p[kStreamArgParts];
    uint32_t n;
};

// The fused FFN's gate/up launch (ah_ffn_gate_up_dev): gate is argument part 0, up part 1 (same
// type and shape, same input); workgroup w serves hidden 32-blocks [w * blocks_per_wg, +blocks_per_wg)
// and writes their SwiGLU, requantized, as the hidden QuantAct.
constexpr uint32_t kFfnMaxBlocks = 16;  // hidden blocks per workgroup (one element per thread)
struct FfnArgs {
    int8_t *h_codes;          // [n_ff]
    int64_t *h_scales;        // [ceil(n_ff / 32)]
    uint32_t n_ff;            // gate / up rows
    uint32_t blocks_per_wg;   // <= kFfnMaxBlocks
};

// GEMM workgroup forms (waves x LDS ring slots), chosen per launch by ah_gemm_pick_waves.
// kFormI8x4 / kFormI8x2: the int8-MFMA design (Q8_0), 4 or 2 waves.
// kFormTile: the dequantize-once design (gemm_dq_kernel: 128 rows x 128 tokens, 4 waves).
// kFormTileFfn: the same tiles over a gate/up pair with the SwiGLU + hidden quantizer epilogue.
enum : uint32_t { kForm4x4 = 0, kForm2x2 = 1, kForm2x4 = 2, kFormI8x4 = 3, kFormI8x2 = 4, kFormTile = 5,
                  kFormTileFfn = 6 };
// The GEMM design of a part: register-blocked f16 (gemm_rb_kernel), int8 (gemm_i8_kernel),
// dequantize-once f16 tiles (gemm_dq_kernel).  Picks its geometry and split model.
enum : uint32_t { kGemmKindRb = 0, kGemmKindI8 = 1, kGemmKindTile = 2 };

// One projection of a GEMM launch: the parts of a launch share the GGUF type, the input and its
// operand (n_in, n_tok), and run in one grid.  `splits` is the part's own split-K count (its
// partials, [splits][n_tok][n_out] f32, are summed by ah_launch_splitk_reduce afterwards).
constexpr uint32_t kGemmMaxParts = 4;
// ah_launch_gemm's `type` for one grid of Q4_K and Q6_K parts (each part's own type applies).
constexpr uint32_t kGemmMixedKQuant = 0xFFFFu;
struct GemmPartDesc {
    const uint8_t *w;
    uint32_t type;    // the part's GGUF type
    uint32_t w_bytes, row_bytes, n_out, splits;
    float *y;         // [n_tok][n_out]
    float *partials;  // with splits > 1
    uint64_t key0;    // added to the part's output refusal keys (t * n_out + row): orders the
                      // refusals of parts that one launch serves (the prefill FFN's gate before up)
};

// The prefill FFN's fused gate/up launch (kFormTileFfn): part 0 is the gate projection, `w_up`
// the up projection of the same type and shape; hidden block rows pair up in the tiles, and the
// epilogue writes the hidden QuantAct instead of the projections' outputs (those optionally).
struct GemmFfn {
    const uint8_t *w_up;
    float *gy, *uy;     // [n_tok][n_ff] f32 gate / up values the SwiGLU consumed, or nullptr
    int8_t *h_codes;    // [n_tok][n_ff]
    int64_t *h_scales;  // [n_tok][ceil(n_ff / 32)]
};

// The unfused prefill FFN's SwiGLU pass over the gate and up projections' f32 outputs.
struct SwigluArgs {
    const float *gate, *up;  // [n_tok][n_ff]
    int8_t *h_codes;         // [n_tok][n_ff]
    int64_t *h_scales;       // [n_tok][ceil(n_ff / 32)]
    uint32_t n_tok, n_ff;
    uint64_t key_sw, key_q;  // refusal key bases: element conversion / SwiGLU, block quantizer
    unsigned long long *status;
};

// The streaming kernel instantiation whose plan mixes GGUF types (each wave dispatches on its
// part's type).
constexpr int kMixedType = 0;

// Streaming GEMV plan: what one workgroup serves.  Each of its 8 waves streams a row range of one
// part; the workgroup quantizes the activation of every part its waves use into its own LDS
// region first.
constexpr uint32_t kIdleWave = 0xFFFFFFFFu;  // wave_part of a wave with no rows
struct StreamWG {
    uint32_t n_act;        // distinct parts (activations) of the workgroup
    uint32_t act_part[8];  // their part indices
    uint32_t act_off[8];   // LDS byte offsets of their activations
    uint32_t wave_part[8]; // per wave: part index, or kIdleWave
    uint32_t wave_act[8];  // per wave: index into act_*
    uint32_t r_begin[8], r_end[8];  // per wave: its rows as one contiguous range of whole tiles
    // per wave, the same count of tiles taken strided (the streaming kernel's form): tiles
    // t_first, t_first + t_stride, ... of its part, so that the part's waves read adjacent tiles
    // at the same time
    uint32_t t_first[8], t_stride[8];
};

// Persistent decode sequence (gemv_seq_kernel): stages run in order on one resident grid, each
// waiting at a grid barrier for the previous stage's outputs.
enum : uint32_t { kSeqGemv = 0, kSeqSwiglu = 1 };
constexpr uint32_t kSeqGroup = 16;   // workgroups per completion counter
constexpr uint32_t kSeqMaxGroups = 64; // one counter per lane of the polling wave: grid <= 1024
constexpr uint32_t kSeqLine = 32;      // u32 words per 128-byte line (one counter per line)
struct SeqStage {
    uint32_t kind;        // kSeqGemv / kSeqSwiglu
    uint32_t wgd_off;     // GEMV: this stage's StreamWG table starts at wgd[wgd_off] (grid entries)
    uint32_t n;           // SwiGLU: hidden width
    uint32_t prod_off;    // producers[prod_off + g]: workgroups of group g with work in this stage
    const float *gate;    // SwiGLU: f32 gate / up outputs of an earlier stage
    const float *up;
    int8_t *codes;        // SwiGLU: the hidden QuantAct (codes [n], scales [ceil(n/32)])
    int64_t *scales;
};
struct SeqArgs {
    const SeqStage *stages;
    const GemvPart *parts;
    const StreamWG *wgd;
    const uint32_t *producers;     // per stage, kSeqMaxGroups producer counts
    unsigned *done;                // per stage and group, a completion counter on its own line
    unsigned *runs;                // per workgroup: launches it has completed
    unsigned long long *status;    // [n_stages]: each stage's first refusal
    uint32_t n_stages, act_bytes;  // LDS activation region of a workgroup (largest stage)
    uint32_t spin_limit;           // polls before a wait gives up (AH_ERR_SEQ_TIMEOUT)
};

// Polls of a persistent sequence's grid-barrier wait before it gives up (about 0.1 s of s_sleep).
constexpr uint32_t kSeqSpinLimit = 1u << 21;
// A wait that gave up records this key, below every refusal key (those hold a status code >= 1 in
// their low byte after an index), so the stage reports AH_ERR_SEQ_TIMEOUT ahead of what its
// workgroups then computed from inputs that were not ready.
constexpr unsigned long long kSeqTimeoutKey = 0ull;

struct QuantArgs {
    const void *x;         // f32 or int64 [n_tok][n_in]
    int8_t *codes;         // [n_tok][n_in]
    int64_t *scales;       // [n_tok][nb32]
    uint32_t n_tok, n_in, nb32;
    uint32_t src;          // AH_SRC_F32 / AH_SRC_Q32
    unsigned long long *status;
};

// GEMM activation operand built from a QuantAct: xh[tok][kpad] f16 = xq * 2^(e_b - E_tok) (exact
// when e_b - E_tok >= -kF16Band), tok_scale[tok] = 2^(E_tok - 32), and for Q4_K the min-term
// operand xmin[tok][kpad/256][16] (split sub-block code sums, see ah_gemm.hip).
//
// A token with a nonzero block below the band (e_b - E_tok < -kF16Band) cannot be carried exactly
// by the f16 operand.  The pass flags it in the lowest mantissa bit of its tok_scale (a power of
// two, so that bit is otherwise 0; readers take the value with ah_ts_value) and, for f32 input,
// keeps its codes and scales (fcodes / fscales rows, written for flagged tokens only).  The GEMM
// then serves flagged tokens from those with exact integer group dots and f32 power-of-two scales,
// as the GEMV does, instead of the MFMA.
constexpr int kF16Band = 24;
AH_DEV float ah_ts_value(uint32_t bits) { return __builtin_bit_cast(float, bits & ~1u); }
AH_DEV bool ah_ts_flagged(uint32_t bits) { return (bits & 1u) != 0; }
struct OperandArgs {
    const void *x;         // f32 / Q32.32 int64 [n_tok][n_in], or int8 codes with `scales`
    const int64_t *scales; // [n_tok][nb32] with AH_SRC_CODES
    _Float16 *xh;          // [n_tok][kpad], or nullptr
    // the same operand in MFMA fragment order, or nullptr: 1 KB per (32-token block tb, 16-K
    // block kb), at ((tb * kpad / 16 + kb) * 64 + lane) * 16 bytes the 8 values K = 16 kb + 8 (lane
    // >> 5) .. +7 of token 32 tb + (lane & 31) -- one coalesced 16-byte load per lane per fragment
    _Float16 *xf;
    float *tok_scale;      // [n_tok] (bit 0: flagged)
    _Float16 *xmin;        // [n_tok][kpad/256][16] for Q4_K, else nullptr
    _Float16 *xmin16;      // [n_tok][kpad/256][16] 16-group code sums X16 * 2^(e_b - E) (|X16| <= 2032:
                           // exact in f16 unsplit) for Q2_K, else nullptr
    int8_t *fcodes;        // [n_tok][n_in] (f32 input only; flagged rows written)
    int64_t *fscales;      // [n_tok][nb32] (f32 input only; flagged rows written)
    int8_t *xc;            // int8 design: codes [n_tok][kpad] (zero past n_in), or nullptr
    uint32_t *xsp;         // int8 design: [n_tok][kpad/32] bf16 pairs of 2^(e_b - E_tok), or nullptr
    uint32_t *xsx;         // int8 Q4_K: [n_tok][kpad/32] 2^(e_b - E_tok) X_b as bf16 (hi, lo), or nullptr
    unsigned long long *status;
    uint32_t n_tok, n_in, nb32, kpad, src;
};
