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
#include "ah_units.h"

namespace {

constexpr uint32_t kThreads = 256;

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
                if (o.xsx) {
                    // Q4_K: 2^(e-E) X_b (|X_b| <= 4064: 12 significant bits) as bf16 hi | lo << 16,
                    // hi + lo exact
                    const float xv = ex[u] < 0 ? 0.0f : __builtin_ldexpf((float)sum[u], ex[u] - E);
                    const uint32_t hi = __builtin_bit_cast(uint32_t, xv) & 0xffff0000u;
                    const uint32_t lo = __builtin_bit_cast(uint32_t, xv - __builtin_bit_cast(float, hi)) & 0xffff0000u;
                    o.xsx[(size_t)tok * nbp + b] = (hi >> 16) | lo;
                }
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
// A part's rows are cut into tiles of whole rows, at most kStreamTile bytes each, and its waves
// take the tiles strided (wave k of n: tiles k, k + n, ...), so the tiles in flight at any time
// are adjacent in memory.  A tile is read with 16-byte buffer loads in which lane l takes chunks
// l, l+64, ... (each load instruction reads 1 KB contiguous; a chunk past the tile takes an
// out-of-range offset and reads nothing), held in registers while the wave computes the previous
// tile from its LDS slot, then written to the slot.  Eight waves share a workgroup and its quantized activation; the tile loop has no
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
    // The wave's rows: tiles t_k, t_k + t_s, t_k + 2 t_s, ... of RW rows each, counted from row
    // r_begin and cut at r_end.  A part's waves take its tiles strided (t_k the wave's index among
    // them, t_s their number), so that at any time they read adjacent tiles of the weights: a bare
    // read at this grid measured 6.2 TB/s against 5.8 with each wave on a contiguous range.
    uint32_t r_begin, r_end, aoff = 0, t_k = 0, t_s = 1;
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
        r_begin = 0;
        r_end = idle ? 0u : P.n_out;
        t_k = D->t_first[wv];
        t_s = D->t_stride[wv];
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
        r_begin = 0;
        r_end = P.n_out;
        t_k = (blockIdx.x - P.wg_begin) * kSWaves + wv;
        t_s = P.wg_count * kSWaves;
    }
    // GEMV parts take f32 or code inputs (the Q32.32 form is the quantizer's alone): telling the
    // compiler drops that form's 16-word inputs from the prologue's registers
    __builtin_assume(P.src != AH_SRC_Q32);
    const uint32_t kpad = (P.n_in + 255) / 256 * 256;
    const ActLds A = carve(smem + aoff, kpad);
    uint8_t *tl = smem + act_bytes + wave * kSlotBytes;
    const __amdgpu_buffer_rsrc_t rs = ah_rsrc(P.w, (uint32_t)P.w_bytes);
    const uint32_t U = P.units, RW = P.rows_per_tile, RB = P.row_bytes, G = P.lanes;
    const uint32_t n_tiles = (r_end - r_begin + RW - 1) / RW;
    const uint32_t n_t = t_k < n_tiles ? (n_tiles - t_k + t_s - 1) / t_s : 0u;

    // Tile t's loads.  All kChunks loads are issued, chunks past the tile out of range (they read
    // nothing), so that the compiler's load counting sees the same loads on every path and never
    // waits for one that is still streaming when it only needs an older one.  A wave requests no
    // tile past its last: the out-of-range loads of an empty tile still take the vector memory
    // path (a decode token took 3% longer with them).
    u32x4 chunk[kChunks];
    auto load_tile = [&](uint32_t t) {
        const uint32_t r0 = r_begin + (t_k + t * t_s) * RW;
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
        const uint32_t r0 = r_begin + (t_k + t * t_s) * RW;
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

// LDS bytes of one part's quantized activation (codes with padding, fsc, fx32, xs16): a multiple
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
