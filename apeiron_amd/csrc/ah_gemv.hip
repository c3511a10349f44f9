// ah_gemv.hip -- decode GEMV (N = 1) over GGUF Q8_0 / Q4_K / Q6_K payloads, and the standalone
// activation quantizer.
//
// Reference semantics: matvec_q8act (chart/mod.rs:1887) equals matvec_fixed on the quantized
// activation; every row is the per-group fold acc += S_b * (w_scale*dot - w_min*xsum)
// (RowAcc::emit, chart/mod.rs:501-514) with exact integer group dots.  Here each dot is exact
// (v_dot4c_i32_i8), and the fold is done in f32 with the activation scale S_b * 2^-32 (a power
// of two, exact in f32) and the f16 weight scales (exact in f32).
//
// Work decomposition (HBM-bound): a row is owned by G = 2^log2g consecutive lanes of a wave; lane
// g of the row walks units g, g+G, ... (Q8_0: one 34-byte block; Q4_K / Q6_K: one 144 / 210-byte
// super-block), loading its unit with 16-byte buffer loads straight from the GGUF bytes.  The
// activation is quantized once per workgroup into LDS (codes, per-32 f32 scale, per-32 and per-16
// code sums), so every lane's activation reads are LDS broadcasts.  Row partials are reduced over
// the G lanes with xor shuffles in a fixed order (deterministic output).
#include "ah_internal.h"

namespace {

constexpr uint32_t kThreads = 256;

struct ActLds {
    int8_t *codes;   // [kpad]
    float *fsc;      // [kpad/32]   S_b * 2^-32
    int32_t *xs32;   // [kpad/32]   sum of codes per 32-block
    int32_t *xs16;   // [kpad/16]   sum of codes per 16-group
};

AH_DEV ActLds carve(uint8_t *smem, uint32_t kpad) {
    ActLds a;
    a.codes = reinterpret_cast<int8_t *>(smem);
    a.fsc = reinterpret_cast<float *>(smem + kpad);
    a.xs32 = reinterpret_cast<int32_t *>(a.fsc + kpad / 32);
    a.xs16 = a.xs32 + kpad / 32;
    return a;
}

// Quantize (or load) the activation of part P into LDS: one 32-block per half-wave.
// Codes past n_in (up to kpad) are zero, so ragged rows need no special case: padded lanes
// contribute nothing to any dot or code sum.
AH_DEV void load_activation(const GemvPart &P, uint32_t kpad, const ActLds &A,
                            unsigned long long *status) {
    const uint32_t hw = threadIdx.x >> 5, hl = threadIdx.x & 31;
    const uint32_t nb32 = (P.n_in + 31) / 32;
    for (uint32_t b = hw; b < kpad / 32; b += kThreads / 32) {
        const uint32_t k = b * 32 + hl;
        int code = 0;
        if (P.src == AH_SRC_CODES) {
            if (k < P.n_in) code = static_cast<const int8_t *>(P.x)[k];
            if (hl == 0) A.fsc[b] = b < nb32 ? (float)P.scales[b] * 0x1p-32f : 0.0f;
        } else {
            uint64_t mag = 0;
            bool neg = false;
            if (k < P.n_in) {
                if (P.src == AH_SRC_F32) {
                    uint32_t bits = static_cast<const uint32_t *>(P.x)[k];
                    int err = ah_to_q32_mag(bits, mag, neg);
                    if (err) {
                        ah_record(status, ((unsigned long long)k << 8) | (unsigned)err);
                        mag = 0;
                    }
                } else {
                    int64_t v = static_cast<const int64_t *>(P.x)[k];
                    neg = v < 0;
                    mag = neg ? 0ull - (uint64_t)v : (uint64_t)v;
                }
            }
            uint64_t am = mag;
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) {
                uint64_t t = __shfl_xor(am, o, 32);
                am = t > am ? t : am;
            }
            const int e = ah_act_scale_exp(am);
            bool bad = e == 63;
            if (e >= 0 && e < 63) code = ah_act_code(mag, neg, e, bad);
            if (bad) {
                ah_record(status, AH_QUANT_ORDER_BASE + ((unsigned long long)b << 8) + 7u);
                code = 0;
            }
            if (hl == 0) A.fsc[b] = (e < 0 || e == 63) ? 0.0f : __builtin_ldexpf(1.0f, e - 32);
        }
        A.codes[k] = (int8_t)code;
        int s = code;
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 32);
        if ((hl & 15) == 0) A.xs16[2 * b + (hl >> 4)] = s;
        s += __shfl_xor(s, 16, 32);
        if (hl == 0) A.xs32[b] = s;
    }
}

// ---- per-family row units ------------------------------------------------------------------

// Q8_0 block b of a row (format/quant.rs:238-250): f16 d at byte 0, 32 int8 codes at 2..33.
// Blocks start 2-byte aligned; the 40-byte window from the 4-aligned address below the block is
// realigned in registers.
AH_DEV float q8_0_unit(__amdgpu_buffer_rsrc_t rs, uint32_t blk, uint32_t b, const ActLds &A,
                       int32_t *dots) {
    const uint32_t base = blk & ~3u, sh = blk & 3u;
    const u32x4 a0 = ah_ld128(rs, base), a1 = ah_ld128(rs, base + 16);
    const uint32_t a2 = ah_ld32(rs, base + 32), a3 = ah_ld32(rs, base + 36);
    const uint32_t w[10] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w, a2, a3};
    const uint32_t d16 = (sh ? (w[0] >> 16) : w[0]) & 0xffffu;
    const uint32_t *xw = reinterpret_cast<const uint32_t *>(A.codes + 32 * b);
    int32_t D = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t c = sh ? w[i + 1] : ah_alignbyte(w[i + 1], w[i], 2);
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
// qs[32*(j/2) + l].  Term per sub-block: S_j * (d*sc_j*D_j - dmin*m_j*X_j).
template <int P>
AH_DEV float q4k_pair(const uint32_t *q, uint32_t s0, uint32_t s1, uint32_t s2, float fd,
                      float fdm, uint32_t g0, uint32_t nb32, const ActLds &A, int32_t *dots) {
    const uint32_t *xl = reinterpret_cast<const uint32_t *>(A.codes + 32 * g0);
    int32_t Dlo = 0, Dhi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        Dlo = ah_sdot4(q[i] & 0x0F0F0F0Fu, xl[i], Dlo);
        Dhi = ah_sdot4((q[i] >> 4) & 0x0F0F0F0Fu, xl[8 + i], Dhi);
    }
    int sl, ml, shh, mh;
    q4k_scale_min<2 * P>(s0, s1, s2, sl, ml);
    q4k_scale_min<2 * P + 1>(s0, s1, s2, shh, mh);
    if (dots) {
        dots[g0] = Dlo;
        if (g0 + 1 < nb32) dots[g0 + 1] = Dhi;  // a ragged row ends on an odd sub-block
    }
    const float tlo = fd * (float)(sl * Dlo) - fdm * (float)(ml * A.xs32[g0]);
    const float thi = fd * (float)(shh * Dhi) - fdm * (float)(mh * A.xs32[g0 + 1]);
    return A.fsc[g0] * tlo + A.fsc[g0 + 1] * thi;
}

AH_DEV float q4_k_unit(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t s, uint32_t nb32,
                       const ActLds &A, int32_t *dots) {
    u32x4 v[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) v[i] = ah_ld128(rs, off + 16 * i);
    const float fd = ah_f16_bits_to_f32(v[0].x & 0xffffu), fdm = ah_f16_bits_to_f32(v[0].x >> 16);
    const uint32_t s0 = v[0].y, s1 = v[0].z, s2 = v[0].w;
    float acc = 0.0f;
    const uint32_t g = 8 * s;
    {
        const uint32_t q[8] = {v[1].x, v[1].y, v[1].z, v[1].w, v[2].x, v[2].y, v[2].z, v[2].w};
        acc += q4k_pair<0>(q, s0, s1, s2, fd, fdm, g, nb32, A, dots);
    }
    if (g + 2 < nb32) {
        const uint32_t q[8] = {v[3].x, v[3].y, v[3].z, v[3].w, v[4].x, v[4].y, v[4].z, v[4].w};
        acc += q4k_pair<1>(q, s0, s1, s2, fd, fdm, g + 2, nb32, A, dots);
    }
    if (g + 4 < nb32) {
        const uint32_t q[8] = {v[5].x, v[5].y, v[5].z, v[5].w, v[6].x, v[6].y, v[6].z, v[6].w};
        acc += q4k_pair<2>(q, s0, s1, s2, fd, fdm, g + 4, nb32, A, dots);
    }
    if (g + 6 < nb32) {
        const uint32_t q[8] = {v[7].x, v[7].y, v[7].z, v[7].w, v[8].x, v[8].y, v[8].z, v[8].w};
        acc += q4k_pair<3>(q, s0, s1, s2, fd, fdm, g + 6, nb32, A, dots);
    }
    return acc;
}

// Q6_K super-block s (format/quant.rs:556-599): ql[128] @0, qh[64] @128, int8 sc[16] @192,
// f16 d @208.  Element 128n + 32t + l = (nibble t/2 of ql[64n + 32(t&1) + l]
// | ((qh[32n + l] >> 2t) & 3) << 4) - 32.  The 210-byte super-blocks are 2-byte aligned; the
// 216-byte window from the 4-aligned address below is realigned in registers.
AH_DEV float q6_k_unit(__amdgpu_buffer_rsrc_t rs, uint32_t addr, uint32_t s, uint32_t nb32,
                       uint32_t nb16, const ActLds &A, int32_t *dots16) {
    const uint32_t base = addr & ~3u, sh = addr & 3u;
    uint32_t w[54];
#pragma unroll
    for (int i = 0; i < 13; ++i) {
        const u32x4 t = ah_ld128(rs, base + 16 * i);
        w[4 * i] = t.x;
        w[4 * i + 1] = t.y;
        w[4 * i + 2] = t.z;
        w[4 * i + 3] = t.w;
    }
    w[52] = ah_ld32(rs, base + 208);
    w[53] = ah_ld32(rs, base + 212);
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
            const uint32_t *xw = reinterpret_cast<const uint32_t *>(A.codes + 32 * g);
            int32_t Dlo = 0, Dhi = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t qlw = V(16 * n + 8 * (t & 1) + i);
                const uint32_t lo4 = t < 2 ? (qlw & 0x0F0F0F0Fu) : ((qlw >> 4) & 0x0F0F0F0Fu);
                const uint32_t u = lo4 | (((qh[i] >> (2 * t)) & 0x03030303u) << 4);
                if (i < 4)
                    Dlo = ah_sdot4(u, xw[i], Dlo);
                else
                    Dhi = ah_sdot4(u, xw[i], Dhi);
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
__global__ void __launch_bounds__(kThreads)
    gemv_kernel(GemvPart single, const GemvPart *__restrict__ parts, uint32_t n_parts,
                uint32_t kpad_max, unsigned long long *status) {
    extern __shared__ __align__(16) uint8_t smem[];
    GemvPart P = single;
    uint32_t wg_count;
    if (parts) {
        uint32_t i = 0;
        while (i + 1 < n_parts && parts[i + 1].wg_begin <= blockIdx.x) ++i;
        P = parts[i];
        wg_count = (i + 1 < n_parts ? parts[i + 1].wg_begin : gridDim.x) - P.wg_begin;
    } else {
        wg_count = gridDim.x;
    }
    const uint32_t wg_local = blockIdx.x - P.wg_begin;
    const uint32_t kpad = (P.n_in + 255) / 256 * 256;
    const ActLds A = carve(smem, kpad_max);
    load_activation(P, kpad, A, status);
    __syncthreads();

    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t G = 1u << P.log2g, g = lane & (G - 1), rr = lane >> P.log2g;
    const uint32_t rows_per_wave = 64u >> P.log2g, rows_per_iter = (kThreads / 64) * rows_per_wave;
    const uint32_t nb32 = (P.n_in + 31) / 32;
    const uint32_t ngroups = TYPE == AH_GGML_Q6_K ? (P.n_in + 15) / 16 : nb32;
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(P.w, (uint32_t)P.w_bytes);

    for (uint32_t rb = wg_local * rows_per_iter; rb < P.n_out; rb += wg_count * rows_per_iter) {
        const uint32_t row = rb + wave * rows_per_wave + rr;
        float acc = 0.0f;
        if (row < P.n_out) {
            const uint32_t rbase = row * P.row_bytes;
            int32_t *dots = P.dots ? P.dots + (size_t)row * ngroups : nullptr;
            if (TYPE == AH_GGML_Q8_0) {
                for (uint32_t b = g; b < nb32; b += G) acc += q8_0_unit(rs, rbase + 34 * b, b, A, dots);
            } else if (TYPE == AH_GGML_Q4_K) {
                const uint32_t nsb = (P.n_in + 255) / 256;
                for (uint32_t s = g; s < nsb; s += G) acc += q4_k_unit(rs, rbase + 144 * s, s, nb32, A, dots);
            } else {
                const uint32_t nsb = (P.n_in + 255) / 256;
                for (uint32_t s = g; s < nsb; s += G) acc += q6_k_unit(rs, rbase + 210 * s, s, nb32, ngroups, A, dots);
            }
        }
        for (uint32_t o = 1; o < G; o <<= 1) acc += __shfl_xor(acc, (int)o, 64);
        if (row < P.n_out && g == 0) P.y[row] = acc;
    }
}

// Standalone quantizer: one token row per workgroup-iteration, one 32-block per half-wave.
// Writes the exact QuantAct (codes, int64 scales) and, optionally, the GEMM operand: codes as
// f16 scaled by 2^(e_b - E) where E is the token's largest block exponent (exact whenever
// e_b - E >= -24), with the token factor 2^(E - 32) stored separately.
__global__ void __launch_bounds__(kThreads) quant_kernel(QuantArgs q) {
    __shared__ int tok_e[kThreads / 32];
    const uint32_t hw = threadIdx.x >> 5, hl = threadIdx.x & 31;
    const uint32_t kpadq = (q.n_in + 31) / 32 * 32;
    for (uint32_t tok = blockIdx.x; tok < q.n_tok; tok += gridDim.x) {
        int emax = -1;
        // pass 1: codes, scales, and the token's largest block exponent
        for (uint32_t b = hw; b < kpadq / 32; b += kThreads / 32) {
            const uint32_t k = b * 32 + hl;
            uint64_t mag = 0;
            bool neg = false;
            int e = -1, code = 0;
            if (q.src == AH_SRC_CODES) {
                int64_t S = q.scales[(size_t)tok * q.nb32 + b];
                e = S > 0 ? 63 - __builtin_clzll((uint64_t)S) : -1;
            } else {
                if (k < q.n_in) {
                    if (q.src == AH_SRC_F32) {
                        uint32_t bits = static_cast<const uint32_t *>(q.x)[(size_t)tok * q.n_in + k];
                        int err = ah_to_q32_mag(bits, mag, neg);
                        if (err) {
                            ah_record(q.status, (((unsigned long long)tok * q.n_in + k) << 8) | (unsigned)err);
                            mag = 0;
                        }
                    } else {
                        int64_t v = static_cast<const int64_t *>(q.x)[(size_t)tok * q.n_in + k];
                        neg = v < 0;
                        mag = neg ? 0ull - (uint64_t)v : (uint64_t)v;
                    }
                }
                uint64_t am = mag;
#pragma unroll
                for (int o = 16; o > 0; o >>= 1) {
                    uint64_t t = __shfl_xor(am, o, 32);
                    am = t > am ? t : am;
                }
                e = ah_act_scale_exp(am);
                bool bad = e == 63;
                if (e >= 0 && e < 63) code = ah_act_code(mag, neg, e, bad);
                if (bad) {
                    ah_record(q.status, AH_QUANT_ORDER_BASE +
                                            (((unsigned long long)tok * q.nb32 + b) << 8) + 7u);
                    code = 0;
                    e = -1;
                }
                if (k < q.n_in) q.codes[(size_t)tok * q.n_in + k] = (int8_t)code;
                if (hl == 0) q.scales[(size_t)tok * q.nb32 + b] = e < 0 ? 0 : (int64_t)(1ull << e);
            }
            emax = e > emax ? e : emax;
        }
        if (q.xh == nullptr) continue;
        // token exponent E = max over blocks
        if (hl == 0) tok_e[hw] = emax;
        __syncthreads();
        int E = -1;
        for (uint32_t i = 0; i < kThreads / 32; ++i) E = tok_e[i] > E ? tok_e[i] : E;
        __syncthreads();
        if (threadIdx.x == 0) q.tok_scale[tok] = E < 0 ? 0.0f : __builtin_ldexpf(1.0f, E - 32);
        // pass 2: f16 operand (codes re-read; same thread wrote them in pass 1)
        for (uint32_t k = threadIdx.x; k < q.kpad; k += kThreads) {
            float v = 0.0f;
            if (k < q.n_in) {
                const int code = q.codes[(size_t)tok * q.n_in + k];
                const int64_t S = q.scales[(size_t)tok * q.nb32 + k / 32];
                if (S > 0) {
                    const int e = 63 - __builtin_clzll((uint64_t)S);
                    v = __builtin_ldexpf((float)code, e - E);
                }
            }
            q.xh[(size_t)tok * q.kpad + k] = (_Float16)v;
        }
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

hipError_t ah_launch_gemv(uint32_t type, const GemvPart &single, const GemvPart *d_parts,
                          uint32_t n_parts, uint32_t grid, uint32_t kpad_max,
                          unsigned long long *status, hipStream_t stream) {
    const size_t lds = kpad_max + (size_t)kpad_max / 32 * 8 + (size_t)kpad_max / 16 * 4;
    switch (type) {
    case AH_GGML_Q8_0:
        hipLaunchKernelGGL(gemv_kernel<AH_GGML_Q8_0>, dim3(grid), dim3(kThreads), lds, stream,
                           single, d_parts, n_parts, kpad_max, status);
        break;
    case AH_GGML_Q4_K:
        hipLaunchKernelGGL(gemv_kernel<AH_GGML_Q4_K>, dim3(grid), dim3(kThreads), lds, stream,
                           single, d_parts, n_parts, kpad_max, status);
        break;
    case AH_GGML_Q6_K:
        hipLaunchKernelGGL(gemv_kernel<AH_GGML_Q6_K>, dim3(grid), dim3(kThreads), lds, stream,
                           single, d_parts, n_parts, kpad_max, status);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t ah_launch_quant(const QuantArgs &q, hipStream_t stream) {
    uint32_t grid = q.n_tok < 1024 ? q.n_tok : 1024;
    if (grid == 0) return hipSuccess;
    hipLaunchKernelGGL(quant_kernel, dim3(grid), dim3(kThreads), 0, stream, q);
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
