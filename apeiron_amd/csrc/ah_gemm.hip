// ah_gemm.hip -- prefill GEMM (N > 1) over GGUF Q8_0 / Q4_K / Q6_K payloads on gfx950 MFMA.
//
// Reference semantics: column c of matmat_q8act (kern/matmat.rs:134) is matvec_q8act on token c;
// the reference's GEMMs (kern/gemm.rs:488-580 Q8_0, chart/kcols.rs:1399-1518 Q4_K / Q6_K) fold
// sum_b d_rb * S_cb * D_rcb with exact integer group dots D.
//
// MI355X design.  A per-32-block f32 epilogue after an int8 MFMA costs ~3 VALU ops per output
// element per block (convert, scale, accumulate), six times the VALU slots a 32x32x32 i8 MFMA
// leaves free.  Instead both operands are fed to v_mfma_f32_32x32x16_f16 as exact small
// integers:
//   * the activation operand is xq * 2^(e_b - E_tok) in f16 (the quantizer's power-of-two block
//     scale S_b = 2^e_b folded in exactly; E_tok is the token's largest block exponent, applied
//     once at the end), so the MFMA itself applies the activation scale;
//   * the weight operand is the integer code (Q8_0 q, Q6_K u-32) or, for Q4_K, sc_j * q (<= 945),
//     exact in f16.
// Every product is exact and every partial sum below 2^24 is exact in the f32 accumulator, so a
// Q8_0 block result is exactly 2^(e_b-E) * D_b.  What remains per output element is one FMA per
// weight-scale change: per 32-block (Q8_0 d), per 16-group (Q6_K d*sc), per 256-super-block
// (Q4_K d, plus one FMA for the dmin*m*X term, which rides on one extra MFMA per super-block).
//
// Tiling: a workgroup is 4 waves; wave w owns 32 weight rows (the MFMA N/column dimension, so
// the weight scale is one value per lane) and all TN = 32*NT tokens of the workgroup (the MFMA M
// dimension).  The f16 activation tile of each 64-deep K stage is staged in LDS and shared by the
// 4 waves; each wave reads its own weight rows straight from the GGUF bytes and converts them in
// registers.  Split-K over grid.z writes partials that a second pass reduces in fixed order.
#include "ah_internal.h"

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kNT = 4;                 // token tiles (of 32) per workgroup
constexpr int kTN = 32 * kNT;          // tokens per workgroup
constexpr int kKS = 64;                // K depth of one LDS stage
constexpr int kPitch = kKS * 2 + 16;   // bytes per token row in LDS (padding breaks bank aliasing)

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

// 4 unsigned 6-bit values (bytes) -> 4 exact f16 of (u - 32).
AH_DEV void u6x4_to_f16(uint32_t u, uint32_t &lo, uint32_t &hi) {
    const f16x2 bias = {(_Float16)1056.0f, (_Float16)1056.0f};
    lo = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
    hi = as_u(as_h2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}

// 4 nibble bytes (values 0..15 in the low nibble of each byte) times sc -> 4 exact f16 sc*q.
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

struct GemmArgs {
    const uint8_t *w;
    uint32_t w_bytes, row_bytes;
    uint32_t n_out, n_in, n_tok, kpad;
    const _Float16 *xh;        // [n_tok][kpad]
    const _Float16 *xmin;      // Q4_K: [n_tok][kpad/256][16] split code sums (see quant pass)
    const float *tok_scale;    // [n_tok]
    float *y;                  // [n_tok][n_out] (splits == 1) or partials [splits][n_tok][n_out]
    uint32_t stages_per_split; // K stages of 64 per split (multiple of the kernel's unroll)
    uint32_t splits;
    uint32_t tok_tiles, n_wg;  // register-blocked grid: token tiles, real workgroup count
};

// The A operand of token tile `tile` for k-offset `kk` (elements) within the stage.
AH_DEV f16x8 act_frag(const uint8_t *lds, int tile, int kk) {
    const int lane = threadIdx.x & 63;
    return *reinterpret_cast<const f16x8 *>(lds + (tile * 32 + (lane & 31)) * kPitch + 2 * kk);
}

constexpr uint32_t kOob = 0xFFFFFFF0u;  // a buffer offset past any operand: reads zeros

// Weight bytes one lane needs for one 64-deep stage, fetched a stage ahead.
//   Q8_0: per block, the lane half's 16 codes (the 4-aligned 20 bytes around them, realigned at
//         use with a register shift -- no per-lane register indexing) and the dword holding d.
//   Q4_K: the super-block header (d, dmin, 12 packed scales) and the lane half's 16 nibble bytes.
struct WStage {
    u32x4 a0, a1, b0, b1;
    uint32_t a2, a3, b2, b3;
};

template <int TYPE>
AH_DEV WStage fetch_w(__amdgpu_buffer_rsrc_t rs, uint32_t rbase, uint32_t st, uint32_t n_in, int h,
                      bool live) {
    WStage w;
    const uint32_t k0 = st * kKS;
    if constexpr (TYPE == AH_GGML_Q8_0) {
        const uint32_t b = k0 / 32;
        const uint32_t blk0 = rbase + 34 * b, blk1 = blk0 + 34;
        const bool l0 = live && b * 32 < n_in, l1 = live && (b + 1) * 32 < n_in;
        const uint32_t c0 = (blk0 + 2 + 16 * h) & ~3u, c1 = (blk1 + 2 + 16 * h) & ~3u;
        w.a0 = ah_ld128_nt(rs, l0 ? c0 : kOob);
        w.a2 = ah_ld32(rs, l0 ? c0 + 16 : kOob);
        w.a3 = ah_ld32(rs, l0 ? (blk0 & ~3u) : kOob);
        w.b0 = ah_ld128_nt(rs, l1 ? c1 : kOob);
        w.b2 = ah_ld32(rs, l1 ? c1 + 16 : kOob);
        w.b3 = ah_ld32(rs, l1 ? (blk1 & ~3u) : kOob);
        w.a1 = w.b1 = (u32x4){0u, 0u, 0u, 0u};
    } else if constexpr (TYPE == AH_GGML_Q4_K) {
        const uint32_t sb = rbase + 144 * (k0 / 256), p = (k0 / 64) & 3;
        w.a0 = ah_ld128(rs, live ? sb : kOob);
        w.a1 = ah_ld128_nt(rs, live ? sb + 16 + 32 * p + 16 * h : kOob);
        w.b0 = w.b1 = (u32x4){0u, 0u, 0u, 0u};
        w.a2 = w.a3 = w.b2 = w.b3 = 0u;
    } else {
        w.a0 = w.a1 = w.b0 = w.b1 = (u32x4){0u, 0u, 0u, 0u};
        w.a2 = w.a3 = w.b2 = w.b3 = 0u;
    }
    return w;
}

// Pipelined K loop.  The [kTN tokens][64 k] f16 activation slice of a stage is shared by the 4
// waves through one of two LDS buffers: while the waves compute stage s from buffer s&1, every
// thread holds stage s+1's slice in registers (loaded during stage s-1) and writes it to the other
// buffer after its MFMAs, then requests stage s+2.  Weight bytes are fetched a stage ahead into
// registers.  One LDS-only barrier per stage; every load is issued unconditionally (out-of-range
// offsets read zeros), so the compiler's load counting never drains the prefetches.
template <int TYPE>
__global__ void __launch_bounds__(kThreads, 2) gemm_kernel(GemmArgs a) {
    __shared__ __align__(16) uint8_t lds[2][kTN * kPitch];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 31, h = lane >> 5;
    const uint32_t row0 = blockIdx.x * 128 + wave * 32;
    const uint32_t tok0 = blockIdx.y * kTN;
    const uint32_t my_row = row0 + j;
    const bool row_ok = my_row < a.n_out;
    const uint32_t rbase = (row_ok ? my_row : 0) * a.row_bytes;
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(a.w, a.w_bytes);
    // this workgroup's token rows of the operand (at most kTN * 32768 * 2 bytes)
    const uint32_t ntile = a.n_tok - tok0 < (uint32_t)kTN ? a.n_tok - tok0 : (uint32_t)kTN;
    const __amdgpu_buffer_rsrc_t rx = ah_rsrc(a.xh + (size_t)tok0 * a.kpad, ntile * a.kpad * 2u);

    const uint32_t nstages = (a.n_in + kKS - 1) / kKS;
    const uint32_t st_begin = blockIdx.z * a.stages_per_split;
    uint32_t st_end = st_begin + a.stages_per_split;
    if (st_end > nstages) st_end = nstages;

    u32x4 areg[kTN * 8 / kThreads];
    auto act_load = [&](uint32_t st) {
        const bool live = st < st_end;
#pragma unroll
        for (int i = 0; i < kTN * 8 / kThreads; ++i) {
            const uint32_t c = threadIdx.x + kThreads * i, t = c >> 3, kc = c & 7;
            const uint32_t off = (t * a.kpad + st * kKS + 8 * kc) * 2u;
            areg[i] = ah_ld128(rx, live && t < ntile ? off : kOob);
        }
    };
    auto act_store = [&](uint8_t *buf) {
#pragma unroll
        for (int i = 0; i < kTN * 8 / kThreads; ++i) {
            const uint32_t c = threadIdx.x + kThreads * i, t = c >> 3, kc = c & 7;
            *reinterpret_cast<u32x4 *>(buf + t * kPitch + 16 * kc) = areg[i];
        }
    };

    f32x16 acc[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) acc[t] = (f32x16){};

    // per-super-block state (K-quants)
    f32x16 P[kNT];
    float fd = 0.0f, fdm = 0.0f;
    uint32_t s0 = 0, s1 = 0, s2 = 0;   // Q4_K packed scales
    uint32_t w6[54];                   // Q6_K super-block window
    uint32_t sh6 = 0;

    act_load(st_begin);
    act_store(lds[0]);
    act_load(st_begin + 1);
    WStage wc = fetch_w<TYPE>(rs, rbase, st_begin, a.n_in, h, st_begin < st_end);

    for (uint32_t st = st_begin; st < st_end; ++st) {
        const uint32_t k0 = st * kKS;
        const uint8_t *cur = lds[(st - st_begin) & 1];
        ah_lds_barrier();  // buffer `cur` is written; every wave is done with the other one
        const WStage wn = fetch_w<TYPE>(rs, rbase, st + 1, a.n_in, h, st + 1 < st_end);
        // keep the next stage's weight requests here, a whole stage ahead of their use (the
        // scheduler would otherwise sink them to the end of the iteration)
        __builtin_amdgcn_sched_barrier(0);

        if (TYPE == AH_GGML_Q8_0) {
            // two 32-blocks per stage; lane half h owns codes [16h, 16h+16) of each block
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                // a block past n_in has zero codes and d = 0 (fetch_w) against zero activations
                const uint32_t b = k0 / 32 + bb;
                const uint32_t blk = rbase + 34 * b;
                const uint32_t shc = (blk + 2 + 16 * h) & 3u;  // 0 or 2
                const u32x4 v = bb ? wc.b0 : wc.a0;
                const uint32_t w[5] = {v.x, v.y, v.z, v.w, bb ? wc.b2 : wc.a2};
                const uint32_t dw = bb ? wc.b3 : wc.a3;
                const float d = ah_f16_bits_to_f32((dw >> (8 * (blk & 3u))) & 0xffffu);
                uint32_t c[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) c[i] = ah_alignbyte(w[i + 1], w[i], shc);
                uint32_t f[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) i8x4_to_f16(c[i], f[2 * i], f[2 * i + 1]);
                const f16x8 b0 = pack8(f[0], f[1], f[2], f[3]), b1 = pack8(f[4], f[5], f[6], f[7]);
#pragma unroll
                for (int t = 0; t < kNT; ++t) {
                    f32x16 p = mfma(act_frag(cur, t, 32 * bb + 16 * h), b0, (f32x16){});
                    p = mfma(act_frag(cur, t, 32 * bb + 16 * h + 8), b1, p);
                    acc[t] += d * p;
                }
            }
        } else if (TYPE == AH_GGML_Q4_K) {
            const uint32_t s = k0 / 256, p = (k0 / 64) & 3;
            if (p == 0) {
                const u32x4 hd = wc.a0;
                fd = ah_f16_bits_to_f32(hd.x & 0xffffu);
                fdm = ah_f16_bits_to_f32(hd.x >> 16);
                s0 = hd.y;
                s1 = hd.z;
                s2 = hd.w;
#pragma unroll
                for (int t = 0; t < kNT; ++t) P[t] = (f32x16){};
            }
            // qs window p: lane half h takes bytes [16h, 16h+16) -> sub-block 2p (low nibbles)
            // and 2p+1 (high nibbles), k = 16h + 8m + e.
            const u32x4 q = wc.a1;
            const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
            int scv[2];
            {
                auto byte = [&](int i) -> uint32_t {
                    const uint32_t wv = i < 4 ? s0 : (i < 8 ? s1 : s2);
                    return (wv >> (8 * (i & 3))) & 0xffu;
                };
#pragma unroll
                for (int hb = 0; hb < 2; ++hb) {
                    const int jj = 2 * (int)p + hb;
                    scv[hb] = jj < 4 ? (int)(byte(jj) & 63)
                                     : (int)((byte(jj + 4) & 0xF) | ((byte(jj - 4) >> 6) << 4));
                }
            }
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                const _Float16 sc = (_Float16)(float)scv[hb];
                const f16x2 sc2 = {sc, sc}, off2 = {(_Float16)(-1024.0f) * sc, (_Float16)(-1024.0f) * sc};
                uint32_t f[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t n = hb ? ((qw[i] >> 4) & 0x0F0F0F0Fu) : (qw[i] & 0x0F0F0F0Fu);
                    nib4_times(n, sc2, off2, f[2 * i], f[2 * i + 1]);
                }
                const f16x8 b0 = pack8(f[0], f[1], f[2], f[3]), b1 = pack8(f[4], f[5], f[6], f[7]);
#pragma unroll
                for (int t = 0; t < kNT; ++t) {
                    P[t] = mfma(act_frag(cur, t, 32 * hb + 16 * h), b0, P[t]);
                    P[t] = mfma(act_frag(cur, t, 32 * hb + 16 * h + 8), b1, P[t]);
                }
            }
            if (p == 3 || k0 + kKS >= a.n_in) {
                // min term: sum_j m_j * X_j over the super-block, one MFMA with K' = 16:
                // A'[tok][8h+e] = split code sum of sub-block e (hi piece h=0, lo piece h=1),
                // B'[8h+e][row] = m_e.
                auto byte = [&](int i) -> uint32_t {
                    const uint32_t wv = i < 4 ? s0 : (i < 8 ? s1 : s2);
                    return (wv >> (8 * (i & 3))) & 0xffu;
                };
                uint32_t mf[4];
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const int m0 = e < 4 ? (int)(byte(e + 4) & 63)
                                         : (int)((byte(e + 4) >> 4) | ((byte(e) >> 6) << 4));
                    const int m1 = e + 1 < 4 ? (int)(byte(e + 5) & 63)
                                             : (int)((byte(e + 5) >> 4) | ((byte(e + 1) >> 6) << 4));
                    const f16x2 mm = {(_Float16)(float)m0, (_Float16)(float)m1};
                    mf[e / 2] = as_u(mm);
                }
                const f16x8 bm = pack8(mf[0], mf[1], mf[2], mf[3]);
                const uint32_t nsb = a.kpad / 256;
#pragma unroll
                for (int t = 0; t < kNT; ++t) {
                    const uint32_t tok = tok0 + 32 * t + j;
                    f16x8 am = {};
                    if (tok < a.n_tok)
                        am = *reinterpret_cast<const f16x8 *>(a.xmin + ((size_t)tok * nsb + s) * 16 + 8 * h);
                    const f32x16 pm = mfma(am, bm, (f32x16){});
                    acc[t] += fd * P[t] - fdm * pm;
                }
            }
        } else {  // Q6_K
            const uint32_t s = k0 / 256, stq = (k0 / 64) & 3;
            if (stq == 0) {
                const uint32_t addr = rbase + 210 * s;
                const uint32_t base = addr & ~3u;
                sh6 = addr & 3u;
#pragma unroll
                for (int i = 0; i < 13; ++i) {
                    const u32x4 t = ah_ld128(rs, base + 16 * i);
                    w6[4 * i] = t.x;
                    w6[4 * i + 1] = t.y;
                    w6[4 * i + 2] = t.z;
                    w6[4 * i + 3] = t.w;
                }
                w6[52] = ah_ld32(rs, base + 208);
                w6[53] = ah_ld32(rs, base + 212);
                fd = ah_f16_bits_to_f32(ah_alignbyte(w6[53], w6[52], sh6) & 0xffffu);
            }
            auto V = [&](int i) -> uint32_t { return ah_alignbyte(w6[i + 1], w6[i], sh6); };
            // stage stq covers elements 64*stq .. +64: half n = stq/2, nibble = stq&1,
            // group G = 4*stq + gg: ql bytes 64n + 16gg + 8h + e, qh bytes 32n + 16(gg&1) + 8h + e,
            // qh shift 2t with t = 2*(stq&1) + gg/2.
            const int n = stq >> 1, nib = stq & 1;
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) {
                // a group past n_in meets zero activations (the operand is zero up to kpad)
                const int G = 4 * (int)stq + gg;
                const int t = 2 * nib + (gg >> 1);
                const int qlb = 64 * n + 16 * gg + 8 * h;          // byte offset, multiple of 8
                const int qhb = 128 + 32 * n + 16 * (gg & 1) + 8 * h;
                uint32_t u[2];
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint32_t qlw = V(qlb / 4 + i), qhw = V(qhb / 4 + i);
                    const uint32_t lo4 = nib ? ((qlw >> 4) & 0x0F0F0F0Fu) : (qlw & 0x0F0F0F0Fu);
                    u[i] = lo4 | (((qhw >> (2 * t)) & 0x03030303u) << 4);
                }
                uint32_t f[4];
                u6x4_to_f16(u[0], f[0], f[1]);
                u6x4_to_f16(u[1], f[2], f[3]);
                const f16x8 bq = pack8(f[0], f[1], f[2], f[3]);
                const uint32_t scw = V(48 + G / 4);
                const float coef = fd * (float)(int)(int8_t)((scw >> (8 * (G & 3))) & 0xffu);
#pragma unroll
                for (int tt = 0; tt < kNT; ++tt) {
                    const f32x16 p = mfma(act_frag(cur, tt, 16 * gg + 8 * h), bq, (f32x16){});
                    acc[tt] += coef * p;
                }
            }
        }

        act_store(lds[((st - st_begin) & 1) ^ 1]);  // stage st+1 (zeros past the split)
        act_load(st + 2);
        wc = wn;
    }

    // D layout of a 32x32 MFMA: lane (j, h), register r -> row i = 8*(r/4) + 4*h + (r%4), col j.
    // Buffer stores relative to this workgroup's token rows; a lane past n_out or a token past
    // n_tok stores out of range (nothing is written), so there is no branch per element.
    float *ybase = a.splits == 1 ? a.y + (size_t)tok0 * a.n_out
                                 : a.y + ((size_t)blockIdx.z * a.n_tok + tok0) * a.n_out;
    const __amdgpu_buffer_rsrc_t ry = ah_rsrc(ybase, ntile * a.n_out * 4u);
    // the token scales of the lane's 16 tokens per tile (1.0 for partials), loaded up front
    const __amdgpu_buffer_rsrc_t rt = ah_rsrc(a.tok_scale + tok0, ntile * 4u);
    const bool scaled = a.splits == 1;
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
        uint32_t sc[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = ah_ld32(rt, 4 * (32 * t + 8 * (r / 4) + 4 * h + (r % 4)));
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t tl = 32 * t + 8 * (r / 4) + 4 * h + (r % 4);
            const bool ok = row_ok && tl < ntile;
            const float v = acc[t][r] * (scaled ? __builtin_bit_cast(float, sc[r]) : 1.0f);
            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry,
                                                  ok ? (tl * a.n_out + my_row) * 4u : kOob, 0, 0);
        }
    }
}


// ---- register-blocked kernel (Q8_0, Q4_K) ---------------------------------------------------
//
// A workgroup is 4 waves.  Wave w owns NN 32-row MFMA column tiles (n) of weight rows and all NM
// 32-token row tiles (m) of the workgroup's tokens, so every activation fragment read from LDS
// feeds NN MFMAs and every dequantized weight fragment feeds NM.  The VALU work per MFMA (weight
// dequantization over NM, plus the scale folds) is what bounds this kernel, so NM = 4 by default;
// LDS sustains the resulting 1 KB of fragment reads per MFMA.  The loop body is U stages of 64
// (Q8_0: U = 2, Q4_K: U = 4 = one super-block), so the LDS buffer, the weight register set and the
// super-block position of each stage are compile-time: no runtime register indexing, no copies
// between register sets.
namespace rb {
constexpr int kNN = 1, kNM = 4;                 // column / row tiles per wave
constexpr int kTok = 32 * kNM;                  // tokens per workgroup
constexpr int kRows = 4 * 32 * kNN;             // weight rows per workgroup
constexpr int kActBytes = kTok * kPitch;        // f16 activation slice of one stage
constexpr int kBufBytes = kActBytes + kTok * 32; // + Q4_K split code sums of the super-block
template <int TYPE> constexpr int unroll() { return TYPE == AH_GGML_Q8_0 ? 2 : 4; }
}  // namespace rb

// Weight bytes of one stage for the lane's NN rows, fetched a stage ahead.  Ordinary (not
// non-temporal) loads: the workgroups of the other token tiles read the same bytes from L2.
//   Q8_0: per row n and block bb, v[2n+bb] = the 16 codes of the lane half (4-aligned window),
//         s[4n+2bb] = the dword after the window, s[4n+2bb+1] = the dword holding d.
//   Q4_K: v[2n] = super-block header (read at the super-block's first stage only),
//         v[2n+1] = the lane half's 16 bytes of qs chunk P.
struct WRb {
    u32x4 v[4];
    uint32_t s[8];
};

template <int TYPE, int P, int NN>
AH_DEV WRb fetch_rb(__amdgpu_buffer_rsrc_t rs, const uint32_t (&rb)[NN], const bool (&rl)[NN],
                    uint32_t st, uint32_t n_in, int h, bool live) {
    WRb w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w.v[i] = (u32x4){0u, 0u, 0u, 0u};
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

template <int TYPE>
__global__ void __launch_bounds__(kThreads, 2) gemm_rb_kernel(GemmArgs a) {
    constexpr int U = rb::unroll<TYPE>(), NN = rb::kNN, NM = rb::kNM;
    __shared__ __align__(16) uint8_t lds[2][rb::kBufBytes];
    // XCD-aware order: dispatch i goes to XCD i % 8, so XCD x takes logical ids
    // [x * per, (x + 1) * per).  Consecutive logical ids share a weight row tile and split, so the
    // workgroups reading the same weights share one XCD's L2.  The grid is a multiple of 8.
    const uint32_t per = gridDim.x >> 3;
    const uint32_t L = (blockIdx.x & 7u) * per + (blockIdx.x >> 3);
    if (L >= a.n_wg) return;  // whole workgroup, before any barrier
    const uint32_t tt = L % a.tok_tiles, rest = L / a.tok_tiles;
    const uint32_t split = rest % a.splits, rtile = rest / a.splits;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 31, h = lane >> 5;
    const uint32_t row_w = rtile * rb::kRows + wave * 32 * NN;
    uint32_t rbase[NN];
    bool rl[NN];
#pragma unroll
    for (int n = 0; n < NN; ++n) {
        const uint32_t r = row_w + 32 * n + j;
        rl[n] = r < a.n_out;
        rbase[n] = (rl[n] ? r : 0u) * a.row_bytes;
    }
    const uint32_t tok0 = tt * rb::kTok;
    const uint32_t ntile = a.n_tok - tok0 < (uint32_t)rb::kTok ? a.n_tok - tok0 : (uint32_t)rb::kTok;
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(a.w, a.w_bytes);
    const __amdgpu_buffer_rsrc_t rx = ah_rsrc(a.xh + (size_t)tok0 * a.kpad, ntile * a.kpad * 2u);
    const uint32_t nsb = a.kpad / 256;
    const __amdgpu_buffer_rsrc_t rm =
        ah_rsrc(TYPE == AH_GGML_Q4_K ? a.xmin + (size_t)tok0 * nsb * 16 : a.xh,
                TYPE == AH_GGML_Q4_K ? ntile * nsb * 32u : 0u);

    // stages: whole super-blocks for Q4_K (zero activations past n_in), pairs for Q8_0
    const uint32_t nstages = TYPE == AH_GGML_Q4_K ? a.kpad / kKS : ((a.n_in + 2 * kKS - 1) / (2 * kKS)) * 2;
    const uint32_t st_begin = split * a.stages_per_split;
    uint32_t st_end = st_begin + a.stages_per_split;
    if (st_end > nstages) st_end = nstages;

    // activation slice of a stage: 32*NM tokens x 128 B = NM 16-B chunks per thread (+ Q4_K: the
    // 32-B split code sums of the stage's super-block, one 16-B chunk per thread of the first NM
    // waves)
    u32x4 areg[NM], mreg;
    auto act_load = [&](uint32_t st) {
        const bool live = st < st_end;
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            const uint32_t c = tid + kThreads * i, t = c >> 3, kc = c & 7;
            areg[i] = ah_ld128(rx, live && t < ntile ? (t * a.kpad + st * kKS + 8 * kc) * 2u : kOob);
        }
        if constexpr (TYPE == AH_GGML_Q4_K) {
            const uint32_t t = (tid >> 1) & (rb::kTok - 1), hc = tid & 1;
            mreg = ah_ld128(rm, live && tid < 2 * rb::kTok && t < ntile ? ((t * nsb + st / 4) * 16 + 8 * hc) * 2u : kOob);
        }
    };
    auto act_store = [&](uint8_t *buf) {
#pragma unroll
        for (int i = 0; i < NM; ++i) {
            const uint32_t c = tid + kThreads * i, t = c >> 3, kc = c & 7;
            *reinterpret_cast<u32x4 *>(buf + t * kPitch + 16 * kc) = areg[i];
        }
        if constexpr (TYPE == AH_GGML_Q4_K) {
            if (tid < 2 * rb::kTok)  // whole waves
                *reinterpret_cast<u32x4 *>(buf + rb::kActBytes + (tid >> 1) * 32 + 16 * (tid & 1)) = mreg;
        }
    };
    auto frag = [&](const uint8_t *buf, int m, int kk) -> f16x8 {
        return *reinterpret_cast<const f16x8 *>(buf + (m * 32 + j) * kPitch + 2 * kk);
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

    act_load(st_begin);
    act_store(lds[0]);
    act_load(st_begin + 1);
    WRb W[2];
    W[0] = fetch_rb<TYPE, 0, NN>(rs, rbase, rl, st_begin, a.n_in, h, st_begin < st_end);

    auto stage = [&](auto uc, uint32_t st) {
        constexpr int u = decltype(uc)::value;
        const uint8_t *cur = lds[u & 1];
        ah_lds_barrier();  // buffer `cur` is written; every wave is done with the other one
        W[(u + 1) & 1] = fetch_rb<TYPE, (u + 1) % U, NN>(rs, rbase, rl, st + 1, a.n_in, h, st + 1 < st_end);
        __builtin_amdgcn_sched_barrier(0);  // the next stage's weight requests stay a stage ahead
        const WRb &wc = W[u & 1];
        if constexpr (TYPE == AH_GGML_Q8_0) {
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
                    const uint32_t blk = rbase[n] + 34 * (st * 2 + bb);
                    const uint32_t shc = (blk + 2 + 16 * h) & 3u;  // 0 or 2
                    const u32x4 v = wc.v[2 * n + bb];
                    const uint32_t w5[5] = {v.x, v.y, v.z, v.w, wc.s[4 * n + 2 * bb]};
                    const uint32_t dw = wc.s[4 * n + 2 * bb + 1];
                    d[bb][n] = ah_f16_bits_to_f32((dw >> (8 * (blk & 3u))) & 0xffffu);
                    uint32_t f[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i) i8x4_to_f16(ah_alignbyte(w5[i + 1], w5[i], shc), f[2 * i], f[2 * i + 1]);
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
                    const _Float16 sc = (_Float16)(float)scv;
                    const f16x2 sc2 = {sc, sc}, off2 = {(_Float16)(-1024.0f) * sc, (_Float16)(-1024.0f) * sc};
                    const u32x4 q = wc.v[2 * n + 1];
                    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
                    uint32_t f[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t nb = hb ? ((qw[i] >> 4) & 0x0F0F0F0Fu) : (qw[i] & 0x0F0F0F0Fu);
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
                        const f16x8 am = *reinterpret_cast<const f16x8 *>(cur + rb::kActBytes + (32 * m + j) * 32 + 16 * h);
                        const f32x16 pm = mfma(am, bm, (f32x16){});
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            acc[m][n][r] = __builtin_fmaf(-fdm[n], pm[r], __builtin_fmaf(fd[n], P[m][n][r], acc[m][n][r]));
                        P[m][n] = (f32x16){};
                    }
                }
            }
        }
        act_store(lds[(u + 1) & 1]);  // stage st+1 (zeros past the split)
        act_load(st + 2);
    };

    for (uint32_t st = st_begin; st < st_end; st += U) {
        stage(std::integral_constant<int, 0>{}, st);
        stage(std::integral_constant<int, 1>{}, st + 1);
        if constexpr (U == 4) {
            stage(std::integral_constant<int, 2>{}, st + 2);
            stage(std::integral_constant<int, 3>{}, st + 3);
        }
    }

    // D layout of a 32x32 MFMA: lane (j, h), register r -> row i = 8*(r/4) + 4*h + (r%4), col j.
    // Token scales (1.0 for partials) are loaded up front; lanes past n_out and tokens past n_tok
    // store out of range, so there is no branch per element.
    float *ybase = a.splits == 1 ? a.y + (size_t)tok0 * a.n_out
                                 : a.y + ((size_t)split * a.n_tok + tok0) * a.n_out;
    const __amdgpu_buffer_rsrc_t ry = ah_rsrc(ybase, ntile * a.n_out * 4u);
    const __amdgpu_buffer_rsrc_t rt = ah_rsrc(a.tok_scale + tok0, ntile * 4u);
    const bool scaled = a.splits == 1;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        uint32_t sc[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[r] = ah_ld32(rt, 4 * (32 * m + 8 * (r / 4) + 4 * h + (r % 4)));
#pragma unroll
        for (int n = 0; n < NN; ++n) {
            const uint32_t row = row_w + 32 * n + j;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t tl = 32 * m + 8 * (r / 4) + 4 * h + (r % 4);
                const bool ok = rl[n] && tl < ntile;
                const float v = acc[m][n][r] * (scaled ? __builtin_bit_cast(float, sc[r]) : 1.0f);
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), ry,
                                                      ok ? (tl * a.n_out + row) * 4u : kOob, 0, 0);
            }
        }
    }
}

// y[tok][row] = tok_scale[tok] * sum_s partial[s][tok][row], fixed summation order.
__global__ void splitk_reduce(const float *part, uint32_t splits, uint32_t n_tok, uint32_t n_out,
                              const float *tok_scale, float *y) {
    const size_t n = (size_t)n_tok * n_out;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        float s = 0.0f;
        for (uint32_t z = 0; z < splits; ++z) s += part[z * n + i];
        y[i] = s * tok_scale[i / n_out];
    }
}

}  // namespace

namespace {

// Stages of 64 the kernel for `type` runs over K, its unroll, and its workgroup tile.
struct GemmGeom {
    uint32_t nstages, unroll, rows, toks;
};
GemmGeom geom_of(uint32_t type, uint32_t n_in, uint32_t kpad) {
    if (type == AH_GGML_Q8_0) return {(n_in + 2 * kKS - 1) / (2 * kKS) * 2, 2, rb::kRows, rb::kTok};
    if (type == AH_GGML_Q4_K) return {kpad / kKS, 4, rb::kRows, rb::kTok};
    return {(n_in + kKS - 1) / kKS, 4, 128, kTN};
}

// Stages per split for a requested split count: a multiple of the unroll.
uint32_t per_split(const GemmGeom &g, uint32_t splits) {
    uint32_t per = (g.nstages + splits - 1) / splits;
    return (per + g.unroll - 1) / g.unroll * g.unroll;
}

}  // namespace

// Split-K count for an n_tok x n_out GEMM on `cus` compute units.  Cost model (microseconds):
// the busiest CU runs ceil(workgroups / cus) workgroups of `per` stages each (~0.25 us a stage),
// and every split beyond the first costs its partials' write and read-back at ~4 TB/s.
uint32_t ah_gemm_pick_splits(uint32_t type, uint32_t n_out, uint32_t n_in, uint32_t n_tok,
                             uint32_t cus) {
    const GemmGeom g = geom_of(type, n_in, (n_in + 255) / 256 * 256);
    const uint64_t tiles = (uint64_t)((n_out + g.rows - 1) / g.rows) * ((n_tok + g.toks - 1) / g.toks);
    uint32_t best = 1;
    double best_cost = 1e30;
    for (uint32_t want = 1; want <= 64 && want <= g.nstages; ++want) {
        const uint32_t per = per_split(g, want);
        const uint32_t used = (g.nstages + per - 1) / per;
        if (used != want) continue;
        const double waves = (double)((tiles * used + cus - 1) / cus);
        double cost = waves * per * 0.25;
        if (used > 1) cost += (double)(used + 1) * n_tok * n_out * 4.0 / 4.0e6;
        if (cost < best_cost) {
            best_cost = cost;
            best = used;
        }
    }
    return best;
}

hipError_t ah_launch_gemm(uint32_t type, const uint8_t *w, uint32_t w_bytes, uint32_t row_bytes,
                          uint32_t n_out, uint32_t n_in, uint32_t n_tok, uint32_t kpad,
                          const _Float16 *xh, const _Float16 *xmin, const float *tok_scale,
                          float *y, float *partials, uint32_t splits, hipStream_t stream) {
    GemmArgs a;
    a.w = w;
    a.w_bytes = w_bytes;
    a.row_bytes = row_bytes;
    a.n_out = n_out;
    a.n_in = n_in;
    a.n_tok = n_tok;
    a.kpad = kpad;
    a.xh = xh;
    a.xmin = xmin;
    a.tok_scale = tok_scale;
    const GemmGeom g = geom_of(type, n_in, kpad);
    const uint32_t per = per_split(g, splits ? splits : 1);
    a.stages_per_split = per;
    a.splits = (g.nstages + per - 1) / per;
    a.y = a.splits == 1 ? y : partials;
    a.tok_tiles = (n_tok + g.toks - 1) / g.toks;
    const uint32_t row_tiles = (n_out + g.rows - 1) / g.rows;
    a.n_wg = row_tiles * a.tok_tiles * a.splits;
    const dim3 rb_grid((a.n_wg + 7) / 8 * 8);
    const dim3 grid(row_tiles, a.tok_tiles, a.splits);
    switch (type) {
    case AH_GGML_Q8_0: hipLaunchKernelGGL(gemm_rb_kernel<AH_GGML_Q8_0>, rb_grid, dim3(kThreads), 0, stream, a); break;
    case AH_GGML_Q4_K: hipLaunchKernelGGL(gemm_rb_kernel<AH_GGML_Q4_K>, rb_grid, dim3(kThreads), 0, stream, a); break;
    case AH_GGML_Q6_K: hipLaunchKernelGGL(gemm_kernel<AH_GGML_Q6_K>, grid, dim3(kThreads), 0, stream, a); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.splits == 1) return e;
    const size_t n = (size_t)n_tok * n_out;
    uint32_t rg = (uint32_t)((n + 255) / 256);
    if (rg > 8192) rg = 8192;
    hipLaunchKernelGGL(splitk_reduce, dim3(rg), dim3(256), 0, stream, partials, a.splits, n_tok, n_out,
                       tok_scale, y);
    return hipGetLastError();
}
