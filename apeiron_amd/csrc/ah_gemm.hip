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
    uint32_t stages_per_split; // K stages of 64 per grid.z slice (multiple of 4 for K-quants)
    uint32_t splits;
};

// Stage the [kTN tokens][64 k] f16 activation slice at k0 into LDS (zeros past n_tok).
AH_DEV void stage_act(const GemmArgs &a, uint32_t tok0, uint32_t k0, uint8_t *lds) {
    for (int c = threadIdx.x; c < kTN * 8; c += kThreads) {
        const int t = c >> 3, kc = c & 7;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (tok0 + t < a.n_tok)
            v = *reinterpret_cast<const u32x4 *>(a.xh + (size_t)(tok0 + t) * a.kpad + k0 + 8 * kc);
        *reinterpret_cast<u32x4 *>(lds + t * kPitch + 16 * kc) = v;
    }
}

// The A operand of token tile `tile` for k-offset `kk` (elements) within the stage.
AH_DEV f16x8 act_frag(const uint8_t *lds, int tile, int kk) {
    const int lane = threadIdx.x & 63;
    return *reinterpret_cast<const f16x8 *>(lds + (tile * 32 + (lane & 31)) * kPitch + 2 * kk);
}

template <int TYPE>
__global__ void __launch_bounds__(kThreads, 2) gemm_kernel(GemmArgs a) {
    __shared__ __align__(16) uint8_t lds[kTN * kPitch];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 31, h = lane >> 5;
    const uint32_t row0 = blockIdx.x * 128 + wave * 32;
    const uint32_t tok0 = blockIdx.y * kTN;
    const uint32_t my_row = row0 + j;
    const bool row_ok = my_row < a.n_out;
    const uint32_t rbase = (row_ok ? my_row : 0) * a.row_bytes;
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(a.w, a.w_bytes);

    const uint32_t nstages = (a.n_in + kKS - 1) / kKS;
    const uint32_t st_begin = blockIdx.z * a.stages_per_split;
    uint32_t st_end = st_begin + a.stages_per_split;
    if (st_end > nstages) st_end = nstages;

    f32x16 acc[kNT];
#pragma unroll
    for (int t = 0; t < kNT; ++t) acc[t] = (f32x16){};

    // per-super-block state (K-quants)
    f32x16 P[kNT];
    float fd = 0.0f, fdm = 0.0f;
    uint32_t s0 = 0, s1 = 0, s2 = 0;   // Q4_K packed scales
    uint32_t w6[54];                   // Q6_K super-block window
    uint32_t sh6 = 0;

    for (uint32_t st = st_begin; st < st_end; ++st) {
        const uint32_t k0 = st * kKS;
        __syncthreads();
        stage_act(a, tok0, k0, lds);
        __syncthreads();

        if (TYPE == AH_GGML_Q8_0) {
            // two 32-blocks per stage; lane half h owns codes [16h, 16h+16) of each block
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                const uint32_t b = k0 / 32 + bb;
                if (b * 32 >= a.n_in) break;
                const uint32_t blk = rbase + 34 * b;
                const uint32_t base = blk & ~3u, sh = blk & 3u;
                const u32x4 v0 = ah_ld128(rs, base), v1 = ah_ld128(rs, base + 16);
                const uint32_t v2 = ah_ld32(rs, base + 32), v3 = ah_ld32(rs, base + 36);
                const uint32_t w[10] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, v2, v3};
                const float d = ah_f16_bits_to_f32(((sh ? (w[0] >> 16) : w[0]) & 0xffffu));
                uint32_t c[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int wi = 4 * h + i;  // code dword index within the block
                    c[i] = sh ? w[wi + 1] : ah_alignbyte(w[wi + 1], w[wi], 2);
                }
                uint32_t f[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) i8x4_to_f16(c[i], f[2 * i], f[2 * i + 1]);
                const f16x8 b0 = pack8(f[0], f[1], f[2], f[3]), b1 = pack8(f[4], f[5], f[6], f[7]);
#pragma unroll
                for (int t = 0; t < kNT; ++t) {
                    f32x16 p = mfma(act_frag(lds, t, 32 * bb + 16 * h), b0, (f32x16){});
                    p = mfma(act_frag(lds, t, 32 * bb + 16 * h + 8), b1, p);
                    acc[t] += d * p;
                }
            }
        } else if (TYPE == AH_GGML_Q4_K) {
            const uint32_t s = k0 / 256, p = (k0 / 64) & 3;
            const uint32_t sb = rbase + 144 * s;
            if (p == 0) {
                const u32x4 hd = ah_ld128(rs, sb);
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
            const u32x4 q = ah_ld128(rs, sb + 16 + 32 * p + 16 * h);
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
                    P[t] = mfma(act_frag(lds, t, 32 * hb + 16 * h), b0, P[t]);
                    P[t] = mfma(act_frag(lds, t, 32 * hb + 16 * h + 8), b1, P[t]);
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
                const int G = 4 * (int)stq + gg;
                if (k0 + 16 * gg >= a.n_in) break;
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
                    const f32x16 p = mfma(act_frag(lds, tt, 16 * gg + 8 * h), bq, (f32x16){});
                    acc[tt] += coef * p;
                }
            }
        }
    }

    // D layout of a 32x32 MFMA: lane (j, h), register r -> row i = 8*(r/4) + 4*h + (r%4), col j.
    if (!row_ok) return;
#pragma unroll
    for (int t = 0; t < kNT; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t tok = tok0 + 32 * t + 8 * (r / 4) + 4 * h + (r % 4);
            if (tok >= a.n_tok) continue;
            const float v = acc[t][r];
            if (a.splits == 1)
                a.y[(size_t)tok * a.n_out + my_row] = v * a.tok_scale[tok];
            else
                a.y[((size_t)blockIdx.z * a.n_tok + tok) * a.n_out + my_row] = v;
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

// GEMM activation operand of one token per workgroup (OperandArgs): E_tok = the largest block
// exponent, tok_scale = 2^(E_tok - 32), xh = xq * 2^(e_b - E_tok) in f16 (exact whenever
// e_b - E_tok >= -24; a smaller block is at most 2^-24 of the token's largest), and for Q4_K the
// min-term operand: per super-block, the 8 sub-block code sums X_j split exactly into f16 pieces
// [64*floor(X/64), X mod 64] * 2^(e_j - E_tok), laid out [hi 0..7, lo 0..7].
__global__ void __launch_bounds__(256) operand_kernel(OperandArgs o) {
    __shared__ int red[256];
    for (uint32_t tok = blockIdx.x; tok < o.n_tok; tok += gridDim.x) {
        const int64_t *sc = o.scales + (size_t)tok * o.nb32;
        int em = -1;
        for (uint32_t b = threadIdx.x; b < o.nb32; b += 256) {
            const int64_t S = sc[b];
            const int e = S > 0 ? 63 - __builtin_clzll((uint64_t)S) : -1;
            em = e > em ? e : em;
        }
        red[threadIdx.x] = em;
        __syncthreads();
        for (uint32_t w = 128; w > 0; w >>= 1) {
            if (threadIdx.x < w) red[threadIdx.x] = red[threadIdx.x] > red[threadIdx.x + w] ? red[threadIdx.x] : red[threadIdx.x + w];
            __syncthreads();
        }
        const int E = red[0];
        __syncthreads();
        if (threadIdx.x == 0) o.tok_scale[tok] = E < 0 ? 0.0f : __builtin_ldexpf(1.0f, E - 32);
        const int8_t *codes = o.codes + (size_t)tok * o.n_in;
        _Float16 *xh = o.xh + (size_t)tok * o.kpad;
        for (uint32_t k = threadIdx.x; k < o.kpad; k += 256) {
            float v = 0.0f;
            if (k < o.n_in) {
                const int64_t S = sc[k / 32];
                if (S > 0) v = __builtin_ldexpf((float)codes[k], 63 - __builtin_clzll((uint64_t)S) - E);
            }
            xh[k] = (_Float16)v;
        }
        if (o.xmin) {
            const uint32_t nsb = o.kpad / 256;
            for (uint32_t g = threadIdx.x; g < nsb * 8; g += 256) {
                float hi = 0.0f, lo = 0.0f;
                if (g < o.nb32 && sc[g] > 0) {
                    int X = 0;
                    for (uint32_t l = 0; l < 32 && g * 32 + l < o.n_in; ++l) X += codes[g * 32 + l];
                    const int ex = 63 - __builtin_clzll((uint64_t)sc[g]) - E;
                    const int xhq = (X >= 0 ? X : X - 63) / 64;  // floor(X / 64)
                    hi = __builtin_ldexpf((float)(64 * xhq), ex);
                    lo = __builtin_ldexpf((float)(X - 64 * xhq), ex);
                }
                _Float16 *m = o.xmin + ((size_t)tok * nsb + g / 8) * 16;
                m[g % 8] = (_Float16)hi;
                m[8 + g % 8] = (_Float16)lo;
            }
        }
        __syncthreads();
    }
}

}  // namespace

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
    const uint32_t nstages = (n_in + kKS - 1) / kKS;
    uint32_t per = (nstages + splits - 1) / splits;
    if (type != AH_GGML_Q8_0) per = (per + 3) / 4 * 4;  // split at super-block boundaries
    a.stages_per_split = per;
    a.splits = (nstages + per - 1) / per;
    a.y = a.splits == 1 ? y : partials;
    dim3 grid((n_out + 127) / 128, (n_tok + kTN - 1) / kTN, a.splits);
    switch (type) {
    case AH_GGML_Q8_0: hipLaunchKernelGGL(gemm_kernel<AH_GGML_Q8_0>, grid, dim3(kThreads), 0, stream, a); break;
    case AH_GGML_Q4_K: hipLaunchKernelGGL(gemm_kernel<AH_GGML_Q4_K>, grid, dim3(kThreads), 0, stream, a); break;
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

uint32_t ah_gemm_splits_used(uint32_t type, uint32_t n_in, uint32_t splits) {
    const uint32_t nstages = (n_in + kKS - 1) / kKS;
    uint32_t per = (nstages + splits - 1) / splits;
    if (type != AH_GGML_Q8_0) per = (per + 3) / 4 * 4;
    return (nstages + per - 1) / per;
}

hipError_t ah_launch_operand(const OperandArgs &o, hipStream_t stream) {
    if (o.n_tok == 0) return hipSuccess;
    const uint32_t grid = o.n_tok < 2048 ? o.n_tok : 2048;
    hipLaunchKernelGGL(operand_kernel, dim3(grid), dim3(256), 0, stream, o);
    return hipGetLastError();
}
