// ah_abi.cpp -- host side of the C ABI declared in include/apeiron_hip.h.
//
// Owns the device context (one HIP stream, a device status word, scratch), validates GGUF
// geometry exactly like matvec_fixed (ops/matvec.rs:160-175), scans f16 block scales for the
// NonFiniteScale refusal (num/dequant.rs:25-41), and plans the kernel launches.
#include "apeiron_hip.h"
#include "ah_internal.h"

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

// launchers (ah_gemv.hip, ah_gemm.hip)
hipError_t ah_launch_gemv(uint32_t type, const GemvPart &single, const GemvPart *d_parts,
                          const uint32_t *d_wg_part, uint32_t grid, uint32_t kpad_max, uint32_t nc,
                          unsigned long long *status, hipStream_t stream);
uint32_t ah_gemv_nc(uint32_t row_bytes);
uint32_t ah_gemv_rows_per_tile(uint32_t row_bytes, uint32_t units);
hipError_t ah_gemv_init_attrs();
bool ah_gemv_stream_geometry(uint32_t type, uint32_t row_bytes, uint32_t units, uint32_t n_out, uint32_t &rows,
                             uint32_t &lanes);
size_t ah_gemv_stream_lds_bytes(uint32_t kpad_max);
size_t ah_gemv_act_bytes(uint32_t kpad);
size_t ah_gemv_stream_slot_bytes();
uint32_t ah_gemv_stream_threads();
int ah_gemv_stream_occupancy(uint32_t type, size_t lds);
hipError_t ah_launch_gemv_stream(uint32_t type, const StreamParts &sp, const GemvPart *d_parts,
                                 const StreamWG *d_wgd, uint32_t grid, uint32_t act_bytes,
                                 unsigned long long *status, hipStream_t stream);
hipError_t ah_launch_quant(const QuantArgs &q, hipStream_t stream);
hipError_t ah_launch_ffn_gate_up(uint32_t type, const StreamParts &sp, const FfnArgs &fa, uint32_t grid,
                                 uint32_t act_bytes, unsigned long long *status, hipStream_t stream);
int ah_ffn_occupancy(uint32_t type, uint32_t kpad);
int ah_gemv_seq_occupancy(uint32_t type, size_t act_bytes);
hipError_t ah_launch_gemv_seq(uint32_t type, const SeqArgs &a, uint32_t grid, hipStream_t stream);
hipError_t ah_launch_scan(const uint8_t *w, uint64_t n_blocks, uint32_t block_bytes, uint32_t off0,
                          uint32_t off1, unsigned long long *d_bad, hipStream_t stream);
hipError_t ah_launch_gemm(uint32_t type, uint32_t n_parts, const GemmPartDesc *parts, uint32_t n_in,
                          uint32_t n_tok, uint32_t kpad, const _Float16 *xh, const _Float16 *xf, const _Float16 *xmin,
                          const _Float16 *xmin16,
                          const float *tok_scale, const int8_t *fcodes, const int64_t *fscales,
                          const int8_t *xc, const uint32_t *xsp, const uint32_t *xsx,
                          unsigned long long *status, uint32_t form, hipStream_t stream,
                          const GemmFfn *ffn = nullptr);
hipError_t ah_launch_splitk_reduce(uint32_t n_parts, const GemmPartDesc *parts, uint32_t n_tok,
                                   const float *tok_scale, unsigned long long *status, hipStream_t stream);
uint32_t ah_gemm_pick_splits(uint32_t type, uint32_t n_out, uint32_t n_in, uint32_t n_tok,
                             uint32_t cus, uint32_t kind);
uint32_t ah_gemm_part_wg4(uint32_t type, uint32_t n_out, uint32_t n_in, uint32_t n_tok, uint32_t splits,
                          uint32_t kind);
uint32_t ah_gemm_max_parts(uint32_t type);
uint32_t ah_gemm_pick_waves(uint32_t type, uint64_t n_wg4, uint32_t cus, bool int8);
hipError_t ah_launch_gemm_operand(const OperandArgs &o, hipStream_t stream);
hipError_t ah_launch_swiglu_quant(const SwigluArgs &a, hipStream_t stream);
hipError_t ah_probe_mfma(uint32_t kind, uint32_t cus, const uint32_t *d_seed, uint32_t *d_sink,
                         hipStream_t stream, double *tops);

// Scratch of ah_gemm_f32_noalloc_dev: device memory the library holds on every GPU it runs on
// until the process ends (a static device array: no allocation per call).  In host code
// `scratch` only names the symbol; its device address is resolved once per context by ah_init
// (hipGetSymbolAddress with the context's device current) and kept in ah_ctx::noalloc.
constexpr size_t kNoAllocScratchBytes = 64ull << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

struct ah_ctx {
    int device = -1;
    uint8_t *noalloc = nullptr;  // this device's copy of `scratch`
    hipStream_t stream = nullptr;
    // Two status words: [0] every call's refusals; [1] the refusals of a fused FFN's down
    // projection, reported only when [0] holds none (the reference refuses the FFN at its first
    // failing step, so a refused hidden activation is never projected).
    unsigned long long *d_status = nullptr;
    int last_hip = 0;
    uint32_t last_bad_bits = 0;  // f16 bits behind the last AH_ERR_NONFINITE_SCALE
    int cu_count = 256;
    uint32_t design[32] = {};  // GEMM design per GGUF type (ah_set_gemm_design; 0 = AUTO)
    void *scratch = nullptr;  // device scratch for GEMM operands / host-form staging
    // the unfused prefill FFN's gate / up outputs when the caller keeps none (grown on demand)
    void *ffn_buf = nullptr;
    size_t ffn_buf_bytes = 0;
    uint32_t ffn_form = AH_FFN_PREFILL_AUTO;  // ah_set_ffn_prefill_form
    size_t scratch_bytes = 0;
    // streaming-GEMV occupancy by (type, LDS bytes): a runtime query per launch costs more host
    // time than a small GEMV takes on the device
    static constexpr int kOccSlots = 16;
    uint32_t occ_key[kOccSlots] = {};
    int occ_val[kOccSlots] = {};
    int occ_n = 0;
};

struct ah_tensor {
    uint32_t type = 0;
    size_t n_out = 0, n_in = 0, row_bytes = 0, bytes = 0;
    uint8_t *d = nullptr;
    bool owned = false;
};

struct ah_gemv_plan {
    uint32_t type = 0, n_parts = 0, grid = 0, kpad_max = 0, nc = 4;
    bool stream = false;  // streaming kernel (else the workgroup-tile kernel)
    bool arg_parts = false;        // streaming, parts in the kernel arguments (sp; no tables)
    StreamParts sp = {};
    uint32_t act_bytes = 0;        // streaming: LDS activation region of a workgroup
    GemvPart *d_parts = nullptr;   // part descriptors
    uint32_t *d_wg_part = nullptr; // workgroup-tile kernel: workgroup -> part index
    StreamWG *d_wgd = nullptr;     // streaming kernel: per-workgroup wave assignment
};

struct ah_seq {
    uint32_t type = 0, grid = 0, n_stages = 0, act_bytes = 0;
    SeqStage *d_stages = nullptr;
    GemvPart *d_parts = nullptr;
    StreamWG *d_wgd = nullptr;
    uint32_t *d_prod = nullptr;   // per stage, producer workgroups of each group
    unsigned *d_done = nullptr;   // per stage and group, a completion counter (128-byte lines)
    unsigned *d_runs = nullptr;   // per workgroup, completed launches
    unsigned long long *d_status = nullptr;
    uint32_t spin_limit = kSeqSpinLimit;  // polls before a grid-barrier wait gives up
};

#define AH_HIP(ctx, call)                                                                       \
    do {                                                                                        \
        hipError_t e_ = (call);                                                                 \
        if (e_ != hipSuccess) {                                                                 \
            if (ctx) (ctx)->last_hip = (int)e_;                                                 \
            return AH_ERR_HIP;                                                                  \
        }                                                                                       \
    } while (0)

namespace {

bool geom(uint32_t t, size_t &qk, size_t &bb) {
    switch (t) {
    case AH_GGML_Q8_0: qk = 32; bb = 34; return true;
    case AH_GGML_Q5_0: qk = 32; bb = 22; return true;
    case AH_GGML_Q2_K: qk = 256; bb = 84; return true;
    case AH_GGML_Q3_K: qk = 256; bb = 110; return true;
    case AH_GGML_Q4_K: qk = 256; bb = 144; return true;
    case AH_GGML_Q6_K: qk = 256; bb = 210; return true;
    default: return false;
    }
}

// matvec_fixed's refusal order: type, then row stride / payload size overflow, then length.
int32_t validate(uint32_t t, size_t raw_len, size_t n_out, size_t n_in, size_t &row_bytes,
                 size_t &need) {
    size_t qk, bb;
    if (!geom(t, qk, bb)) return AH_ERR_UNSUPPORTED_QUANT;
    const size_t blocks = n_in / qk + (n_in % qk != 0);
    if (__builtin_mul_overflow(blocks, bb, &row_bytes)) return AH_ERR_LENGTH_OVERFLOW;
    if (__builtin_mul_overflow(n_out, row_bytes, &need)) return AH_ERR_LENGTH_OVERFLOW;
    if (raw_len < need) return AH_ERR_SHORT_PAYLOAD;
    // Device limits of this backend: 32-bit buffer ranges and the LDS-resident activation.
    if (need >= 0xFFFFFF00ull || n_in > AH_MAX_N_IN || n_out >= (1ull << 31)) return AH_ERR_INVALID_ARG;
    return AH_OK;
}

void scale_offsets(uint32_t t, uint32_t &o0, uint32_t &o1, uint32_t &bb) {
    if (t == AH_GGML_Q8_0) { o0 = o1 = 0; bb = 34; }
    else if (t == AH_GGML_Q5_0) { o0 = o1 = 0; bb = 22; }
    else if (t == AH_GGML_Q2_K) { o0 = 80; o1 = 82; bb = 84; }
    else if (t == AH_GGML_Q3_K) { o0 = o1 = 108; bb = 110; }
    else if (t == AH_GGML_Q4_K) { o0 = 0; o1 = 2; bb = 144; }
    else { o0 = o1 = 208; bb = 210; }
}

bool f16_nonfinite(uint16_t h) { return ((h >> 10) & 0x1f) == 0x1f; }

hipStream_t pick(ah_ctx *ctx, void *stream) {
    return stream ? static_cast<hipStream_t>(stream) : ctx->stream;
}

int32_t ensure_scratch(ah_ctx *ctx, size_t bytes) {
    if (bytes <= ctx->scratch_bytes) return AH_OK;
    if (ctx->scratch) {
        // the old scratch may still be read by queued kernels
        AH_HIP(ctx, hipDeviceSynchronize());
        AH_HIP(ctx, hipFree(ctx->scratch));
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
    }
    size_t want = bytes + (bytes >> 2) + 4096;
    if (hipMalloc(&ctx->scratch, want) != hipSuccess) {
        ctx->scratch = nullptr;
        return AH_ERR_OUT_OF_MEMORY;
    }
    ctx->scratch_bytes = want;
    return AH_OK;
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Work units of a row: Q8_0 / Q5_0 blocks, Q4_K super-blocks (or, with `pairs`, sub-block pairs
// of 64 elements), Q2_K / Q3_K / Q6_K half super-blocks (128 elements).
uint32_t units_per_row(uint32_t t, uint32_t n_in, bool pairs = false) {
    return ah_blk32((int)t)        ? (n_in + 31) / 32
           : t == AH_GGML_Q4_K     ? (pairs ? (n_in + 63) / 64 : (n_in + 255) / 256)
                                   : (n_in + 127) / 128;
}
// A streaming Q4_K part of a latency launch (a single projection, a plan of argument parts, a
// decode sequence) whose super-block geometry leaves fewer tiles than this takes pair units: it
// then has idle lanes and CUs to spread its super-blocks over.  A large part's waves are already
// busy, and a table plan (many projections at once) is bound by throughput, where pairs would
// only add their per-pair scale work: those keep super-block units.
constexpr uint32_t kQ4kPairTiles = 512;

uint32_t kpad_of(size_t n_in) { return (uint32_t)((n_in + 255) / 256 * 256); }

// Two kernels serve the GEMV.  The streaming kernel (rows up to one 8 KB tile) deals a part's
// tiles of whole rows to its waves; the workgroup-tile kernel serves longer rows.  make_part fills
// a part's geometry; deal_wgs then sizes every part's workgroup count.

GemvPart make_part(const ah_tensor *w, uint32_t src, const void *x, const int64_t *scales, float *y,
                   int32_t *dots, bool &stream, bool latency = true) {
    GemvPart P;
    std::memset(&P, 0, sizeof(P));
    P.w = w->d;
    P.w_bytes = w->bytes;
    P.x = x;
    P.scales = scales;
    P.y = y;
    P.dots = dots;
    P.n_out = (uint32_t)w->n_out;
    P.n_in = (uint32_t)w->n_in;
    P.row_bytes = (uint32_t)w->row_bytes;
    P.units = units_per_row(w->type, P.n_in);
    uint32_t rows = 0, lanes = 0;
    stream = ah_gemv_stream_geometry(w->type, P.row_bytes, P.units, P.n_out, rows, lanes);
    if (latency && stream && w->type == AH_GGML_Q4_K && P.n_in > 64 && (P.n_out + rows - 1) / rows < kQ4kPairTiles) {
        P.units = units_per_row(w->type, P.n_in, true);
        stream = ah_gemv_stream_geometry(w->type, P.row_bytes, P.units, P.n_out, rows, lanes);
    }
    if (stream) {
        P.rows_per_tile = rows;
        P.lanes = lanes;
    } else {
        P.rows_per_tile = ah_gemv_rows_per_tile(P.row_bytes, P.units);
        P.lanes = 0;
    }
    P.src = src;
    P.type = w->type;
    return P;
}

// Re-cut a part for the workgroup-tile kernel (a plan whose parts do not all stream).
void recut_wg_tiles(GemvPart &P) {
    P.rows_per_tile = ah_gemv_rows_per_tile(P.row_bytes, P.units);
    P.lanes = 0;
}

// Workgroups that are resident on the whole device at once for the kernel serving these parts:
// a launch never asks for more, so no workgroup waits for another to finish before it starts.
uint64_t resident_wgs(ah_ctx *ctx, uint32_t type, bool stream, uint32_t kpad_max) {
    int occ = 4;
    if (stream) {
        const size_t lds = ah_gemv_stream_lds_bytes(kpad_max);
        const uint32_t key = (type << 24) | (uint32_t)lds | 0x800000u;  // lds < 2^23
        occ = -1;
        for (int i = 0; i < ctx->occ_n; ++i)
            if (ctx->occ_key[i] == key) occ = ctx->occ_val[i];
        if (occ < 0) {
            occ = ah_gemv_stream_occupancy(type, lds);
            if (occ > 0 && ctx->occ_n < ah_ctx::kOccSlots) {
                ctx->occ_key[ctx->occ_n] = key;
                ctx->occ_val[ctx->occ_n++] = occ;
            }
        }
    }
    if (occ < 1) occ = 1;
    return (uint64_t)occ * (uint64_t)ctx->cu_count;
}

// Deal `target` workgroups over the parts: one each, then one at a time to the part with the most
// tiles per workgroup, never past one tile per wave (streaming) or per workgroup.  A tile is one
// step of a wave's pipeline whatever its byte count (its arithmetic is one unit per lane), so
// tiles, not bytes, measure a part's time: rows that fit a tile twice (e.g. K = 4864 Q4_K rows
// in 8 KB tiles) make more, smaller tiles per byte.  Returns the grid size (wg_begin / wg_count
// filled), or 0 when the host is out of memory.
uint32_t deal_wgs(GemvPart *parts, size_t n, uint64_t target, bool stream) {
    struct Item {
        double load;
        uint32_t i;
    };
    // argument-part launches (up to 4 parts) keep the heap on the stack: the no-alloc GEMM's
    // Q2_K / Q3_K route comes through here
    Item local[4];
    Item *heap = n <= 4 ? local : static_cast<Item *>(std::malloc(n * sizeof(Item)));
    if (!heap) return 0;
    size_t hn = 0;
    auto tiles_of = [](const GemvPart &P) -> double {
        return (double)((P.n_out + P.rows_per_tile - 1) / P.rows_per_tile);
    };
    auto cap_of = [&](const GemvPart &P) -> uint32_t {
        const uint32_t tiles = (P.n_out + P.rows_per_tile - 1) / P.rows_per_tile;
        const uint32_t wv = ah_gemv_stream_threads() / 64;
        const uint32_t c = stream ? (tiles + wv - 1) / wv : tiles;
        return c ? c : 1u;
    };
    auto push = [&](Item it) {
        size_t k = hn++;
        while (k && heap[(k - 1) / 2].load < it.load) {
            heap[k] = heap[(k - 1) / 2];
            k = (k - 1) / 2;
        }
        heap[k] = it;
    };
    auto pop = [&]() {
        const Item top = heap[0], last = heap[--hn];
        size_t k = 0;
        for (;;) {
            size_t c = 2 * k + 1;
            if (c >= hn) break;
            if (c + 1 < hn && heap[c + 1].load > heap[c].load) ++c;
            if (heap[c].load <= last.load) break;
            heap[k] = heap[c];
            k = c;
        }
        if (hn) heap[k] = last;
        return top;
    };
    uint64_t used = n;
    for (size_t i = 0; i < n; ++i) {
        parts[i].wg_count = 1;
        if (cap_of(parts[i]) > 1) push({tiles_of(parts[i]), (uint32_t)i});
    }
    while (used < target && hn) {
        const Item it = pop();
        GemvPart &P = parts[it.i];
        ++P.wg_count;
        ++used;
        if (P.wg_count < cap_of(P)) push({tiles_of(P) / P.wg_count, it.i});
    }
    if (heap != local) std::free(heap);
    uint32_t wg = 0;
    for (size_t i = 0; i < n; ++i) {
        parts[i].wg_begin = wg;
        wg += parts[i].wg_count;
    }
    return wg;
}

// Streaming plan: deal the waves of `n_wg` resident workgroups over the parts so that the most
// tiles any wave streams is as small as it can be (every part gets at least one wave; a part
// never gets more waves than tiles), then lay the waves out in part order, eight per workgroup.
// A workgroup quantizes the activation of every part its waves use into its own LDS region, so
// a workgroup takes at most 8 parts and `act_budget` bytes of activations: a part that would
// overflow it starts the next workgroup (the waves skipped are idle).  Wave k of a part with n
// waves gets the contiguous tiles [T*k/n, T*(k+1)/n) (r_begin / r_end, the persistent
// sequence's form) and, for the streaming kernel, the same count of tiles strided: k, k + n, ...
// (t_first / t_stride).  Returns the workgroup count (0: does not fit).
uint32_t deal_waves(const GemvPart *parts, size_t n, uint32_t n_wg, size_t act_budget, StreamWG *out) {
    const uint64_t W = (uint64_t)n_wg * 8;
    if (n > W) return 0;
    uint32_t *nw = static_cast<uint32_t *>(std::malloc(n * sizeof(uint32_t)));
    if (!nw) return 0;
    auto tiles = [&](size_t p) { return (parts[p].n_out + parts[p].rows_per_tile - 1) / parts[p].rows_per_tile; };
    auto actb = [&](size_t p) { return ah_gemv_act_bytes(kpad_of(parts[p].n_in)); };
    // Relative time of a wave tile: a Q6_K tile (heavier unpacking) takes ~9/8 of the others
    // (measured on separate Q4_K and Q6_K plans: ~6.1 against ~5.4 us per tile and wave).  In a
    // single-type plan the weight cancels.
    auto tile_w = [&](size_t p) -> uint64_t { return parts[p].type == AH_GGML_Q6_K ? 9u : 8u; };
    uint64_t target = W;
    uint32_t used_wg = 0;
    for (int attempt = 0; attempt < 8 && target >= n; ++attempt) {
        // waves per part: greedy on the largest weighted ceil(tiles / waves)
        uint64_t total = n;
        for (size_t p = 0; p < n; ++p) nw[p] = 1;
        while (total < target) {
            size_t best = n;
            uint64_t bl = 0;
            for (size_t p = 0; p < n; ++p) {
                if (nw[p] >= tiles(p)) continue;
                const uint64_t l = (uint64_t)((tiles(p) + nw[p] - 1) / nw[p]) * tile_w(p);
                if (l > bl) {
                    bl = l;
                    best = p;
                }
            }
            if (best == n) break;  // every part has a wave per tile
            ++nw[best];
            ++total;
        }
        // lay out, eight waves per workgroup
        uint64_t c = 0;
        size_t cur_bytes = 0;
        uint32_t cur_nact = 0;
        bool fits = true;
        for (size_t p = 0; p < n && fits; ++p) {
            const size_t a = actb(p);
            for (uint32_t k = 0; k < nw[p]; ++k) {
                if (c % 8 == 0) {  // a new workgroup starts with this part
                    cur_bytes = 0;
                    cur_nact = 0;
                }
                if (k == 0 || c % 8 == 0) {
                    if (c % 8 != 0 && (cur_bytes + a > act_budget || cur_nact == 8)) {
                        c = (c / 8 + 1) * 8;  // pad: this part starts the next workgroup
                        cur_bytes = 0;
                        cur_nact = 0;
                    }
                    if (a > act_budget) {
                        fits = false;
                        break;
                    }
                    cur_bytes += a;
                    ++cur_nact;
                }
                const uint64_t wg = c / 8, wi = c % 8;
                if (wg >= n_wg) {
                    fits = false;
                    break;
                }
                StreamWG &D = out[wg];
                if (wi == 0 || k == 0) {
                    if (wi == 0) {
                        std::memset(&D, 0, sizeof(D));
                        for (int i = 0; i < 8; ++i) {
                            D.wave_part[i] = kIdleWave;
                            D.t_stride[i] = 1;  // an idle wave streams no tiles (its row range is empty)
                        }
                    }
                    D.act_part[D.n_act] = (uint32_t)p;
                    D.act_off[D.n_act] = D.n_act ? D.act_off[D.n_act - 1] + (uint32_t)actb(D.act_part[D.n_act - 1]) : 0u;
                    ++D.n_act;
                }
                const uint32_t T = tiles(p), RW = parts[p].rows_per_tile;
                const uint32_t tb = (uint32_t)((uint64_t)T * k / nw[p]), te = (uint32_t)((uint64_t)T * (k + 1) / nw[p]);
                D.wave_part[wi] = (uint32_t)p;
                D.wave_act[wi] = D.n_act - 1;
                D.r_begin[wi] = tb * RW < parts[p].n_out ? tb * RW : parts[p].n_out;
                D.r_end[wi] = te * RW < parts[p].n_out ? te * RW : parts[p].n_out;
                D.t_first[wi] = k;
                D.t_stride[wi] = nw[p];
                ++c;
            }
        }
        if (fits) {
            used_wg = (uint32_t)((c + 7) / 8);
            // workgroups whose tail waves were skipped by padding: those waves stay idle
            break;
        }
        target -= target / 16 + 1;  // padding overflowed the grid: fewer waves, try again
    }
    std::free(nw);
    return used_wg;
}

int32_t gemv_launch(ah_ctx *ctx, const ah_tensor *w, uint32_t src, const void *x,
                    const int64_t *scales, float *y, int32_t *dots, void *stream,
                    unsigned long long *status = nullptr, uint32_t key_tok = 0, uint64_t out_key0 = 0) {
    if (ctx && !status) status = ctx->d_status;
    if (!ctx || !w || (!x && w->n_in) || (!y && w->n_out)) return AH_ERR_INVALID_ARG;
    if (src == AH_SRC_CODES && !scales && w->n_in) return AH_ERR_INVALID_ARG;
    // the kernels read codes a dword at a time, f32 / Q32.32 values at their natural alignment
    const uintptr_t align = src == AH_SRC_CODES ? 4 : src == AH_SRC_F32 ? 4 : 8;
    if (reinterpret_cast<uintptr_t>(x) % align || (scales && reinterpret_cast<uintptr_t>(scales) % 8))
        return AH_ERR_INVALID_ARG;
    if (w->n_out == 0) return AH_OK;
    bool st = false;
    StreamParts sp = {};
    sp.n = 1;
    GemvPart &P = sp.p[0];
    P = make_part(w, src, x, scales, y, dots, st);
    P.key_tok = key_tok;
    P.out_key0 = out_key0;
    const uint32_t kp = kpad_of(w->n_in);
    AH_HIP(ctx, hipSetDevice(ctx->device));
    const uint32_t grid = deal_wgs(&P, 1, resident_wgs(ctx, w->type, st, kp), st);
    if (grid == 0) return AH_ERR_OUT_OF_MEMORY;
    if (st)
        AH_HIP(ctx, ah_launch_gemv_stream(w->type, sp, nullptr, nullptr, grid, (uint32_t)ah_gemv_act_bytes(kp),
                                          status, pick(ctx, stream)));
    else
        AH_HIP(ctx, ah_launch_gemv(w->type, P, nullptr, nullptr, grid, kp, ah_gemv_nc(P.row_bytes),
                                   status, pick(ctx, stream)));
    return AH_OK;
}

int32_t reset_status(ah_ctx *ctx) {
    const unsigned long long none[2] = {AH_ST_NONE, AH_ST_NONE};
    AH_HIP(ctx, hipMemcpy(ctx->d_status, none, sizeof(none), hipMemcpyHostToDevice));
    return AH_OK;
}

// GEMM operand preparation + launch.  src = AH_SRC_F32 (x = f32 [n_tok][n_in]) or AH_SRC_CODES.
// Prefill over n_parts projections of one input: one operand pass (shared by every part, as the
// reference's grouped GEMM shares one activation pack, kern/gemm.rs:799-818), then one GEMM launch
// per run of consecutive parts of one GGUF type (up to kGemmMaxParts; Q8_0 one), then one split-K reduction
// for every part that splits.  Each part keeps the split count it would get alone, so its outputs
// are those of its single-projection call bit for bit.  All parts share n_in; types and n_out may
// differ.  A single projection is the group of one.
// `fixed` (with `fixed_cap` bytes) replaces the context's growable scratch: the call then neither
// allocates nor frees anything (device or host, for up to kStackParts parts), and refuses with
// AH_ERR_SCRATCH_LIMIT when its operands and partials need more than `fixed_cap`.
// Output refusals are keyed part by part (part i's key t * n_out_i + row offset by the n_tok *
// n_out of every part before it: the first refusal in projection-then-column-then-row order, as
// separate calls joined left to right would return it; the prefill FFN's gate before its up).
// `opt` (optional): explicit per-part key offsets in place of those, the status word the call
// records into, and the fused FFN form (parts {gate, up} of one dequantize-once type: one launch
// whose epilogue writes the hidden QuantAct; `y` then names the optional f32 gate / up outputs).
constexpr size_t kStackParts = 16;
struct GroupOpts {
    const uint64_t *key0 = nullptr;
    unsigned long long *status = nullptr;
    const GemmFfn *ffn = nullptr;
};
int32_t gemm_group_launch(ah_ctx *ctx, size_t n_parts, const ah_tensor *const *w, uint32_t src,
                          const void *x, const int64_t *scales_in, size_t n_tok, float *const *y,
                          void *stream, uint8_t *fixed = nullptr, size_t fixed_cap = 0,
                          const GroupOpts *opt = nullptr) {
    if (!ctx || !w || !y || n_parts == 0 || n_parts > 65536 || !w[0]) return AH_ERR_INVALID_ARG;
    const GemmFfn *ffn = opt ? opt->ffn : nullptr;
    unsigned long long *const status = opt && opt->status ? opt->status : ctx->d_status;
    uint64_t k0_stack[kStackParts];
    std::vector<uint64_t> k0_heap;
    if (n_parts > kStackParts && !(opt && opt->key0)) {
        if (fixed) return AH_ERR_INVALID_ARG;
        k0_heap.resize(n_parts);
    }
    uint64_t *const k0_own = n_parts > kStackParts ? k0_heap.data() : k0_stack;
    const uint64_t *const key0 = opt && opt->key0 ? opt->key0 : k0_own;
    if (!(opt && opt->key0)) {
        uint64_t acc = 0;
        for (size_t i = 0; i < n_parts; ++i) {
            k0_own[i] = acc;
            acc += w[i] ? (uint64_t)n_tok * w[i]->n_out : 0u;
        }
    }
    const size_t n_in_sz = w[0]->n_in;
    bool any_q4k = false;
    if (ffn && (n_parts != 2 || !w[1] || w[0]->type != w[1]->type || w[0]->n_out != w[1]->n_out))
        return AH_ERR_INVALID_ARG;
    for (size_t i = 0; i < n_parts; ++i) {
        if (!w[i] || (!ffn && !y[i] && w[i]->n_out) || w[i]->n_in != n_in_sz) return AH_ERR_INVALID_ARG;
        // a workgroup's output rows (128 tokens x n_out f32) are addressed with 32-bit offsets
        if (w[i]->n_out > (0xFFFFFF00ull / (128 * 4))) return AH_ERR_INVALID_ARG;
        any_q4k = any_q4k || w[i]->type == AH_GGML_Q4_K;
    }
    if (!x && n_tok && n_in_sz) return AH_ERR_INVALID_ARG;
    if (n_tok == 0) return AH_OK;
    if (n_tok >= (1ull << 24)) return AH_ERR_INVALID_ARG;
    // The design of each part's type (ah_set_gemm_design): Q8_0 and Q4_K parts take the int8-MFMA
    // design when it is selected, the operand pass then writing int8 codes and block factors (for
    // Q4_K also the scaled code sums; the f16 operand only if another part needs it); Q4_K parts
    // may take the dequantize-once tiles.
    auto kind_of = [&](uint32_t type) -> uint32_t {
        if (ffn) return kGemmKindTile;  // the fused FFN form runs on the dequantize-once tiles
        const uint32_t d = type < 32 ? ctx->design[type] : 0u;
        if ((type == AH_GGML_Q8_0 || type == AH_GGML_Q4_K) && d == AH_GEMM_DESIGN_INT8) return kGemmKindI8;
        if (type == AH_GGML_Q4_K && d == AH_GEMM_DESIGN_F16_TILE) return kGemmKindTile;
        // Q2_K / Q3_K: the tiles are their only MFMA design (AH_GEMM_DESIGN_F16 keeps the
        // per-token GEMV route)
        if (ah_k23((int)type) && d != AH_GEMM_DESIGN_F16) return kGemmKindTile;
        return kGemmKindRb;
    };
    // Q2_K / Q3_K parts whose design is AH_GEMM_DESIGN_F16 take GEMV launches of a few tokens
    // each, as matmat_q8act serves these families one column at a time (kern/matmat.rs:392-413);
    // the other parts then go through the GEMM below.  Nothing is allocated on this route (parts
    // past kStackParts aside).  By default these families take the dequantize-once MFMA tiles.
    auto gemv23 = [&](const ah_tensor *t) { return ah_k23((int)t->type) && kind_of(t->type) != kGemmKindTile; };
    size_t n23 = 0;
    for (size_t i = 0; i < n_parts; ++i) n23 += gemv23(w[i]) ? 1 : 0;
    if (n23) {
        const size_t nb = (n_in_sz + 31) / 32;
        // the GEMV reads codes a dword at a time: token rows of codes whose length is not a multiple
        // of 4 are first copied to 4-byte aligned rows of the context scratch (same stream, so the
        // GEMM below may reuse the scratch after these launches)
        size_t pitch = src == AH_SRC_F32 ? n_in_sz * 4 : n_in_sz;
        const int8_t *codes = static_cast<const int8_t *>(x);
        if (src == AH_SRC_CODES && n_in_sz % 4) {
            if (fixed) return AH_ERR_INVALID_ARG;
            pitch = (n_in_sz + 3) & ~(size_t)3;
            int32_t st = ensure_scratch(ctx, n_tok * pitch);
            if (st) return st;
            AH_HIP(ctx, hipSetDevice(ctx->device));
            AH_HIP(ctx, hipMemcpy2DAsync(ctx->scratch, pitch, x, n_in_sz, n_in_sz, n_tok, hipMemcpyDeviceToDevice,
                                         pick(ctx, stream)));
            codes = static_cast<const int8_t *>(ctx->scratch);
        }
        auto x_of = [&](size_t c) -> const void * {
            return src == AH_SRC_F32 ? static_cast<const void *>(static_cast<const float *>(x) + c * n_in_sz)
                                     : static_cast<const void *>(codes + c * pitch);
        };
        const uint32_t kp = kpad_of(n_in_sz);
        AH_HIP(ctx, hipSetDevice(ctx->device));
        for (size_t i = 0; i < n_parts; ++i) {
            if (!gemv23(w[i]) || w[i]->n_out == 0) continue;
            // rows that fit the streaming kernel's tile: four tokens per launch, as the argument
            // parts of one launch (each workgroup quantizes its own token's activation), so each
            // launch fills more of the device and the weight rows are re-read from L2
            bool stream_ok = false;
            (void)make_part(w[i], src, x_of(0), nullptr, y[i], nullptr, stream_ok);
            for (size_t c = 0; c < n_tok;) {
                if (!stream_ok) {
                    const int32_t st = gemv_launch(ctx, w[i], src, x_of(c), src == AH_SRC_CODES ? scales_in + c * nb : nullptr,
                                                   y[i] + c * w[i]->n_out, nullptr, stream, status, (uint32_t)c,
                                                   key0[i] + (uint64_t)c * w[i]->n_out);
                    if (st) return st;
                    ++c;
                    continue;
                }
                StreamParts sp = {};
                sp.n = (uint32_t)(n_tok - c < 4 ? n_tok - c : 4);
                for (uint32_t j = 0; j < sp.n; ++j) {
                    bool st_j = false;
                    sp.p[j] = make_part(w[i], src, x_of(c + j), src == AH_SRC_CODES ? scales_in + (c + j) * nb : nullptr,
                                        y[i] + (c + j) * w[i]->n_out, nullptr, st_j);
                    sp.p[j].key_tok = (uint32_t)(c + j);
                    sp.p[j].out_key0 = key0[i] + (uint64_t)(c + j) * w[i]->n_out;
                }
                const uint32_t grid = deal_wgs(sp.p, sp.n, resident_wgs(ctx, w[i]->type, true, kp), true);
                if (grid == 0) return AH_ERR_OUT_OF_MEMORY;
                AH_HIP(ctx, ah_launch_gemv_stream(w[i]->type, sp, nullptr, nullptr, grid,
                                                  (uint32_t)ah_gemv_act_bytes(kp), status, pick(ctx, stream)));
                c += sp.n;
            }
        }
        if (n23 == n_parts) return AH_OK;
        const ah_tensor *rw_stack[kStackParts];
        float *ry_stack[kStackParts];
        std::vector<const ah_tensor *> rw_heap;
        std::vector<float *> ry_heap;
        if (n_parts > kStackParts) {
            if (fixed) return AH_ERR_INVALID_ARG;
            rw_heap.resize(n_parts);
            ry_heap.resize(n_parts);
        }
        const ah_tensor **rw = n_parts > kStackParts ? rw_heap.data() : rw_stack;
        float **ry = n_parts > kStackParts ? ry_heap.data() : ry_stack;
        size_t k = 0;
        for (size_t i = 0; i < n_parts; ++i)
            if (!gemv23(w[i])) {
                rw[k] = w[i];
                ry[k++] = y[i];
            }
        // the remaining parts keep their key offsets
        GroupOpts o2 = opt ? *opt : GroupOpts{};
        uint64_t t_stack[kStackParts];
        std::vector<uint64_t> t_heap;
        if (n_parts > kStackParts) t_heap.resize(n_parts);
        uint64_t *t0 = n_parts > kStackParts ? t_heap.data() : t_stack;
        size_t q = 0;
        for (size_t i = 0; i < n_parts; ++i)
            if (!gemv23(w[i])) t0[q++] = key0[i];
        o2.key0 = t0;
        return gemm_group_launch(ctx, k, rw, src, x, scales_in, n_tok, ry, stream, fixed, fixed_cap, &o2);
    }
    const uint32_t n_in = (uint32_t)n_in_sz, N = (uint32_t)n_tok;
    const uint32_t kpad = kpad_of(n_in), nb32 = (n_in + 31) / 32, nsb = kpad / 256;
    const uint32_t cus = (uint32_t)ctx->cu_count;
    bool any_int8 = false, any_f16 = false, any_tile = false, any_i8q4 = false;
    for (size_t i = 0; i < n_parts; ++i) {
        const uint32_t k = kind_of(w[i]->type);
        any_int8 = any_int8 || k == kGemmKindI8;
        any_i8q4 = any_i8q4 || (k == kGemmKindI8 && w[i]->type == AH_GGML_Q4_K);
        any_f16 = any_f16 || k == kGemmKindRb;
        any_tile = any_tile || k == kGemmKindTile;
    }
    // every split part has its own partials region: the parts of a launch run together and the
    // reduction reads them all at the end
    GemmPartDesc pd_stack[kStackParts];
    size_t off_stack[kStackParts] = {};
    std::vector<GemmPartDesc> pd_heap;
    std::vector<size_t> off_heap;
    if (n_parts > kStackParts) {
        if (fixed) return AH_ERR_INVALID_ARG;
        pd_heap.resize(n_parts);
        off_heap.assign(n_parts, 0);
    }
    GemmPartDesc *pd = n_parts > kStackParts ? pd_heap.data() : pd_stack;
    size_t *part_off = n_parts > kStackParts ? off_heap.data() : off_stack;
    size_t part_bytes = 0;
    for (size_t i = 0; i < n_parts; ++i) {
        GemmPartDesc &d = pd[i];
        d.w = w[i]->d;
        d.type = w[i]->type;
        d.w_bytes = (uint32_t)w[i]->bytes;
        d.row_bytes = (uint32_t)w[i]->row_bytes;
        d.n_out = (uint32_t)w[i]->n_out;
        d.splits = d.n_out && !ffn ? ah_gemm_pick_splits(w[i]->type, d.n_out, n_in, N, cus, kind_of(w[i]->type)) : 1;
        d.y = y[i];
        d.partials = nullptr;
        d.key0 = key0[i];
        if (d.splits > 1) {
            part_off[i] = part_bytes;
            part_bytes = align256(part_bytes + (size_t)d.splits * N * d.n_out * 4);
        }
    }

    size_t off = 0;
    const size_t o_xh = off; off = align256(off + (any_f16 ? (size_t)N * kpad * 2 : 0));
    // fragment order: whole 32-token blocks (the rows past n_tok are never stored from)
    const size_t o_xf = off; off = align256(off + (any_tile ? (size_t)((N + 31) / 32 * 32) * kpad * 2 : 0));
    const size_t o_xc = off; off = align256(off + (any_int8 ? (size_t)N * kpad : 0));
    const size_t o_xsp = off; off = align256(off + (any_int8 ? (size_t)N * (kpad / 32) * 4 : 0));
    const size_t o_xsx = off; off = align256(off + (any_i8q4 ? (size_t)N * (kpad / 32) * 4 : 0));
    const size_t o_ts = off; off = align256(off + (size_t)N * 4);
    const size_t o_xmin = off; off = align256(off + (any_q4k ? (size_t)N * nsb * 32 : 0));
    bool any_k23 = false;
    for (size_t i = 0; i < n_parts; ++i) any_k23 = any_k23 || ah_k23((int)w[i]->type);
    const size_t o_xmin16 = off; off = align256(off + (any_k23 ? (size_t)N * nsb * 32 : 0));
    // flagged tokens' QuantAct (f32 input; codes input is read in place)
    const bool keep = src == AH_SRC_F32;
    const size_t o_fc = off; off = align256(off + (keep ? (size_t)N * n_in : 0));
    const size_t o_fs = off; off = align256(off + (keep ? (size_t)N * nb32 * 8 : 0));
    const size_t o_part = off; off = align256(off + part_bytes);
    uint8_t *S = fixed;
    if (fixed) {
        if (off > fixed_cap) return AH_ERR_SCRATCH_LIMIT;
    } else {
        const int32_t st = ensure_scratch(ctx, off);
        if (st) return st;
        S = static_cast<uint8_t *>(ctx->scratch);
    }
    _Float16 *xh = any_f16 ? reinterpret_cast<_Float16 *>(S + o_xh) : nullptr;
    _Float16 *xf = any_tile ? reinterpret_cast<_Float16 *>(S + o_xf) : nullptr;
    int8_t *xc = any_int8 ? reinterpret_cast<int8_t *>(S + o_xc) : nullptr;
    uint32_t *xsp = any_int8 ? reinterpret_cast<uint32_t *>(S + o_xsp) : nullptr;
    uint32_t *xsx = any_i8q4 ? reinterpret_cast<uint32_t *>(S + o_xsx) : nullptr;
    float *ts = reinterpret_cast<float *>(S + o_ts);
    _Float16 *xmin = reinterpret_cast<_Float16 *>(S + o_xmin);
    _Float16 *xmin16 = any_k23 ? reinterpret_cast<_Float16 *>(S + o_xmin16) : nullptr;
    int8_t *fcodes = keep ? reinterpret_cast<int8_t *>(S + o_fc) : static_cast<int8_t *>(const_cast<void *>(x));
    int64_t *fscales = keep ? reinterpret_cast<int64_t *>(S + o_fs) : const_cast<int64_t *>(scales_in);
    for (size_t i = 0; i < n_parts; ++i)
        if (pd[i].splits > 1) pd[i].partials = reinterpret_cast<float *>(S + o_part + part_off[i]);
    hipStream_t s = pick(ctx, stream);
    AH_HIP(ctx, hipSetDevice(ctx->device));

    // one pass from the input (or the codes) to the MFMA operand
    OperandArgs o;
    o.x = x;
    o.scales = scales_in;
    o.xh = xh;
    o.xf = xf;
    o.tok_scale = ts;
    o.xmin = any_q4k ? xmin : nullptr;
    o.xmin16 = xmin16;
    o.fcodes = keep ? fcodes : nullptr;
    o.fscales = keep ? fscales : nullptr;
    o.xc = xc;
    o.xsp = xsp;
    o.xsx = xsx;
    o.status = status;
    o.n_tok = N;
    o.n_in = n_in;
    o.nb32 = nb32;
    o.kpad = kpad;
    o.src = src;
    AH_HIP(ctx, ah_launch_gemm_operand(o, s));
    if (ffn) {
        if (pd[0].n_out == 0) return AH_OK;
        AH_HIP(ctx, ah_launch_gemm(w[0]->type, 1, pd, n_in, N, kpad, xh, xf, xmin, xmin16, ts, fcodes, fscales, xc, xsp, xsx,
                                   status, kFormTileFfn, s, ffn));
        return AH_OK;
    }
    // runs of consecutive parts of one type (parts with no rows skipped)
    bool any_split = false;
    for (size_t i = 0; i < n_parts;) {
        if (pd[i].n_out == 0) {
            ++i;
            continue;
        }
        uint32_t type = w[i]->type;
        GemmPartDesc run[kGemmMaxParts];
        uint32_t nr = 0;
        uint64_t wg4 = 0;
        if (kind_of(type) == kGemmKindTile) {
            // dequantize-once tiles: runs of up to four parts of this type
            for (; i < n_parts && nr < kGemmMaxParts; ++i) {
                if (pd[i].n_out == 0) continue;
                if (w[i]->type != type) break;
                run[nr++] = pd[i];
                any_split = any_split || pd[i].splits > 1;
            }
            AH_HIP(ctx, ah_launch_gemm(type, nr, run, n_in, N, kpad, xh, xf, xmin, xmin16, ts, fcodes, fscales, xc, xsp, xsx,
                                       status, kFormTile, s));
            continue;
        }
        // K-quant parts of both types (q/k beside v) share one grid when together they leave CUs
        // idle: one run of consecutive Q4_K/Q6_K parts, if it holds both types and its 4-wave
        // grid is at most two workgroups per CU; otherwise runs of one type
        if (type == AH_GGML_Q4_K || type == AH_GGML_Q6_K) {
            uint32_t k = 0, types = 0;
            uint64_t g4 = 0;
            for (size_t j = i; j < n_parts && k < kGemmMaxParts; ++j) {
                if (pd[j].n_out == 0) continue;
                if (w[j]->type != AH_GGML_Q4_K && w[j]->type != AH_GGML_Q6_K) break;
                if (kind_of(w[j]->type) != kGemmKindRb) break;
                types |= w[j]->type == AH_GGML_Q4_K ? 1u : 2u;
                g4 += ah_gemm_part_wg4(w[j]->type, pd[j].n_out, n_in, N, pd[j].splits, kGemmKindRb);
                ++k;
            }
            if (types == 3u && g4 <= 2ull * cus) type = kGemmMixedKQuant;
        }
        // (an int8 launch takes one part)
        const uint32_t max_run = type == kGemmMixedKQuant ? kGemmMaxParts
                                 : kind_of(type) == kGemmKindI8 ? 1u : ah_gemm_max_parts(type);
        for (; i < n_parts && nr < max_run; ++i) {
            if (pd[i].n_out == 0) continue;
            const bool fits = type == kGemmMixedKQuant
                                  ? ((w[i]->type == AH_GGML_Q4_K || w[i]->type == AH_GGML_Q6_K) &&
                                     kind_of(w[i]->type) == kGemmKindRb)
                                  : w[i]->type == type;
            if (!fits) break;
            run[nr++] = pd[i];
            wg4 += ah_gemm_part_wg4(w[i]->type, pd[i].n_out, n_in, N, pd[i].splits, kind_of(w[i]->type));
            any_split = any_split || pd[i].splits > 1;
        }
        const uint32_t form = type == kGemmMixedKQuant
                                  ? kForm4x4
                                  : ah_gemm_pick_waves(type, wg4, cus, kind_of(type) == kGemmKindI8);
        AH_HIP(ctx, ah_launch_gemm(type, nr, run, n_in, N, kpad, xh, xf, xmin, xmin16, ts, fcodes, fscales, xc, xsp, xsx,
                                   status, form, s));
    }
    if (any_split) AH_HIP(ctx, ah_launch_splitk_reduce((uint32_t)n_parts, pd, N, ts, status, s));
    return AH_OK;
}

int32_t gemm_launch(ah_ctx *ctx, const ah_tensor *w, uint32_t src, const void *x,
                    const int64_t *scales_in, size_t n_tok, float *y, void *stream) {
    if (!ctx || !w || !y || (!x && n_tok && w->n_in)) return AH_ERR_INVALID_ARG;
    if (n_tok == 0 || w->n_out == 0) return AH_OK;
    return gemm_group_launch(ctx, 1, &w, src, x, scales_in, n_tok, &y, stream);
}

}  // namespace

extern "C" {

const char *ah_status_str(int32_t s) {
    switch (s) {
    case AH_OK: return "ok";
    case AH_ERR_SHAPE_MISMATCH: return "shape mismatch";
    case AH_ERR_ROW_LENGTH: return "row length";
    case AH_ERR_SHORT_PAYLOAD: return "short payload";
    case AH_ERR_LENGTH_OVERFLOW: return "length overflow";
    case AH_ERR_UNSUPPORTED_QUANT: return "unsupported quant";
    case AH_ERR_NONFINITE_SCALE: return "non-finite scale";
    case AH_ERR_FIXED_OVERFLOW: return "fixed overflow";
    case AH_ERR_ACCUMULATOR_OVERFLOW: return "accumulator overflow";
    case AH_ERR_OUTPUT_OVERFLOW: return "output overflow";
    case AH_ERR_NONFINITE_INPUT: return "non-finite input";
    case AH_ERR_INPUT_RANGE: return "input out of range";
    case AH_ERR_NO_DEVICE: return "no gfx950 device";
    case AH_ERR_INVALID_ARG: return "invalid argument";
    case AH_ERR_HIP: return "hip error";
    case AH_ERR_OUT_OF_MEMORY: return "out of device memory";
    case AH_ERR_SCRATCH_LIMIT: return "call needs more than the fixed scratch of the no-alloc entry point";
    case AH_ERR_SEQ_TIMEOUT: return "sequence barrier timed out";
    case AH_ERR_FFN_OVERFLOW: return "FFN overflow";
    case AH_ERR_EXP_RANGE: return "exp out of range";
    case AH_ERR_ZERO_DENOMINATOR: return "zero denominator";
    default: return "unknown status";
    }
}

int32_t ah_init(int32_t device, ah_ctx **out) {
    if (!out) return AH_ERR_INVALID_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= device || device < 0) return AH_ERR_NO_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return AH_ERR_NO_DEVICE;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return AH_ERR_NO_DEVICE;
    ah_ctx *ctx = new (std::nothrow) ah_ctx();
    if (!ctx) return AH_ERR_OUT_OF_MEMORY;
    ctx->device = device;
    ctx->cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    if (hipSetDevice(device) != hipSuccess || hipStreamCreate(&ctx->stream) != hipSuccess ||
        hipMalloc(&ctx->d_status, 2 * sizeof(unsigned long long)) != hipSuccess ||
        ah_gemv_init_attrs() != hipSuccess) {
        delete ctx;
        return AH_ERR_HIP;
    }
    void *sp = nullptr;
    const hipError_t se = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));  // this device's copy
    if (se != hipSuccess || !sp || reset_status(ctx) != AH_OK) {
        ctx->last_hip = (int)se;
        (void)hipFree(ctx->d_status);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return AH_ERR_HIP;
    }
    ctx->noalloc = static_cast<uint8_t *>(sp);
    *out = ctx;
    return AH_OK;
}

int32_t ah_destroy(ah_ctx *ctx) {
    if (!ctx) return AH_ERR_INVALID_ARG;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->ffn_buf) (void)hipFree(ctx->ffn_buf);
    (void)hipFree(ctx->d_status);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return AH_OK;
}

int32_t ah_last_hip_error(const ah_ctx *ctx) { return ctx ? ctx->last_hip : 0; }

int32_t ah_last_refusal_bits(const ah_ctx *ctx, uint32_t *bits) {
    if (!ctx || !bits) return AH_ERR_INVALID_ARG;
    *bits = ctx->last_bad_bits;
    return AH_OK;
}

int32_t ah_upload_weight(ah_ctx *ctx, uint32_t type, const void *raw, size_t raw_len, size_t n_out,
                         size_t n_in, ah_tensor **out) {
    if (!ctx || !out || (!raw && raw_len)) return AH_ERR_INVALID_ARG;
    *out = nullptr;
    size_t row_bytes, need;
    int32_t st = validate(type, raw_len, n_out, n_in, row_bytes, need);
    if (st) return st;
    uint32_t o0, o1, bb;
    scale_offsets(type, o0, o1, bb);
    const uint8_t *b = static_cast<const uint8_t *>(raw);
    for (size_t off = 0; off < need; off += bb) {
        const uint16_t h0 = (uint16_t)(b[off + o0] | (b[off + o0 + 1] << 8));
        const uint16_t h1 = (uint16_t)(b[off + o1] | (b[off + o1 + 1] << 8));
        if (f16_nonfinite(h0) || f16_nonfinite(h1)) {
            ctx->last_bad_bits = f16_nonfinite(h0) ? h0 : h1;
            return AH_ERR_NONFINITE_SCALE;
        }
    }
    // A Q4_K row whose K is not a multiple of 256 ends in a partial super-block whose trailing qs
    // chunks the product never reads; the device copy keeps each row's leading `stride` bytes only
    // (16-byte aligned).  The last unit of a row then reads into the next row, or past the tensor,
    // against zero activations: the kernels' LDS tiles carry the slack for it.
    size_t stride = row_bytes;
    if (type == AH_GGML_Q4_K && n_in % 256 && n_in <= 8192)
        stride = 144 * (n_in / 256) + 16 + 32 * ((n_in % 256 + 63) / 64);
    const size_t dev_bytes = n_out * stride;
    const void *src = raw;
    uint8_t *packed = nullptr;
    if (stride != row_bytes) {
        packed = static_cast<uint8_t *>(std::malloc(dev_bytes ? dev_bytes : 1));
        if (!packed) return AH_ERR_OUT_OF_MEMORY;
        for (size_t r = 0; r < n_out; ++r) std::memcpy(packed + r * stride, b + r * row_bytes, stride);
        src = packed;
    }
    ah_tensor *t = new (std::nothrow) ah_tensor();
    if (!t) {
        std::free(packed);
        return AH_ERR_OUT_OF_MEMORY;
    }
    AH_HIP(ctx, hipSetDevice(ctx->device));
    if (hipMalloc(&t->d, dev_bytes + 256) != hipSuccess) {
        std::free(packed);
        delete t;
        return AH_ERR_OUT_OF_MEMORY;
    }
    const hipError_t ce = hipMemcpy(t->d, src, dev_bytes, hipMemcpyHostToDevice);
    std::free(packed);
    if (ce != hipSuccess) {
        (void)hipFree(t->d);
        delete t;
        return AH_ERR_HIP;
    }
    t->type = type;
    t->n_out = n_out;
    t->n_in = n_in;
    t->row_bytes = stride;
    t->bytes = dev_bytes;
    t->owned = true;
    *out = t;
    return AH_OK;
}

int32_t ah_wrap_weight_dev(ah_ctx *ctx, uint32_t type, const void *d_raw, size_t raw_len, size_t n_out,
                           size_t n_in, ah_tensor **out) {
    if (!ctx || !out || (!d_raw && raw_len)) return AH_ERR_INVALID_ARG;
    *out = nullptr;
    size_t row_bytes, need;
    int32_t st = validate(type, raw_len, n_out, n_in, row_bytes, need);
    if (st) return st;
    uint32_t o0, o1, bb;
    scale_offsets(type, o0, o1, bb);
    AH_HIP(ctx, hipSetDevice(ctx->device));
    unsigned long long *d_bad = nullptr;
    AH_HIP(ctx, hipMalloc(&d_bad, sizeof(*d_bad)));
    unsigned long long bad = ~0ull;  // earliest non-finite scale: (block << 17) | (dmin << 16) | bits
    hipError_t e = hipMemcpy(d_bad, &bad, sizeof(bad), hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = ah_launch_scan(static_cast<const uint8_t *>(d_raw), need / bb, bb, o0, o1, d_bad, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = hipMemcpy(&bad, d_bad, sizeof(bad), hipMemcpyDeviceToHost);
    (void)hipFree(d_bad);
    if (e != hipSuccess) {
        ctx->last_hip = (int)e;
        return AH_ERR_HIP;
    }
    if (bad != ~0ull) {
        ctx->last_bad_bits = (uint32_t)(bad & 0xffffu);
        return AH_ERR_NONFINITE_SCALE;
    }
    ah_tensor *t = new (std::nothrow) ah_tensor();
    if (!t) return AH_ERR_OUT_OF_MEMORY;
    t->type = type;
    t->n_out = n_out;
    t->n_in = n_in;
    t->row_bytes = row_bytes;
    t->bytes = need;
    t->d = static_cast<uint8_t *>(const_cast<void *>(d_raw));
    t->owned = false;
    *out = t;
    return AH_OK;
}

int32_t ah_free_tensor(ah_ctx *ctx, ah_tensor *t) {
    if (!ctx || !t) return AH_ERR_INVALID_ARG;
    if (t->owned && t->d) {
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(t->d);
    }
    delete t;
    return AH_OK;
}

int32_t ah_tensor_info(const ah_tensor *t, uint32_t *type, size_t *n_out, size_t *n_in,
                       size_t *row_bytes, const void **d_raw) {
    if (!t) return AH_ERR_INVALID_ARG;
    if (type) *type = t->type;
    if (n_out) *n_out = t->n_out;
    if (n_in) *n_in = t->n_in;
    if (row_bytes) *row_bytes = t->row_bytes;
    if (d_raw) *d_raw = t->d;
    return AH_OK;
}

static int32_t quant_dev(ah_ctx *ctx, uint32_t src, const void *d_x, size_t n_tok, size_t n_in,
                         int8_t *d_codes, int64_t *d_scales, void *stream) {
    if (!ctx || ((!d_x || !d_codes || !d_scales) && n_tok && n_in)) return AH_ERR_INVALID_ARG;
    if (n_tok == 0 || n_in == 0) return AH_OK;
    if (n_in >= (1ull << 31) || n_tok >= (1ull << 31)) return AH_ERR_INVALID_ARG;
    QuantArgs q;
    q.x = d_x;
    q.codes = d_codes;
    q.scales = d_scales;
    q.n_tok = (uint32_t)n_tok;
    q.n_in = (uint32_t)n_in;
    q.nb32 = (uint32_t)((n_in + 31) / 32);
    q.src = src;
    q.status = ctx->d_status;
    AH_HIP(ctx, hipSetDevice(ctx->device));
    AH_HIP(ctx, ah_launch_quant(q, pick(ctx, stream)));
    return AH_OK;
}

int32_t ah_quant_act_f32_dev(ah_ctx *ctx, const float *d_x, size_t n_tok, size_t n_in,
                             int8_t *d_codes, int64_t *d_scales, void *stream) {
    return quant_dev(ctx, AH_SRC_F32, d_x, n_tok, n_in, d_codes, d_scales, stream);
}

int32_t ah_quant_act_q32_dev(ah_ctx *ctx, const int64_t *d_x, size_t n_tok, size_t n_in,
                             int8_t *d_codes, int64_t *d_scales, void *stream) {
    return quant_dev(ctx, AH_SRC_Q32, d_x, n_tok, n_in, d_codes, d_scales, stream);
}

int32_t ah_gemv_f32_dev(ah_ctx *ctx, const ah_tensor *w, const float *d_x, float *d_y, void *stream) {
    return gemv_launch(ctx, w, AH_SRC_F32, d_x, nullptr, d_y, nullptr, stream);
}

int32_t ah_gemv_q8_dev(ah_ctx *ctx, const ah_tensor *w, const int8_t *d_codes,
                       const int64_t *d_scales, float *d_y, void *stream) {
    return gemv_launch(ctx, w, AH_SRC_CODES, d_codes, d_scales, d_y, nullptr, stream);
}

int32_t ah_gemv_q8_dots_dev(ah_ctx *ctx, const ah_tensor *w, const int8_t *d_codes,
                            const int64_t *d_scales, float *d_y, int32_t *d_dots, void *stream) {
    if (!d_dots) return AH_ERR_INVALID_ARG;
    return gemv_launch(ctx, w, AH_SRC_CODES, d_codes, d_scales, d_y, d_dots, stream);
}

// The decode FFN's gate/up launch from an f32 input (src AH_SRC_F32) or a QuantAct (AH_SRC_CODES:
// x = codes, 4-byte aligned, with `scales`).
static int32_t ffn_gate_up_launch(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, uint32_t src,
                                  const void *d_x, const int64_t *d_scales, float *d_gate_y, float *d_up_y,
                                  int8_t *d_h_codes, int64_t *d_h_scales, void *stream) {
    if (!ctx || !gate || !up || !d_x || !d_h_codes || !d_h_scales) return AH_ERR_INVALID_ARG;
    if (src == AH_SRC_CODES && (!d_scales || reinterpret_cast<uintptr_t>(d_scales) % 8)) return AH_ERR_INVALID_ARG;
    if (gate->type != up->type || gate->n_out != up->n_out || gate->n_in != up->n_in || gate->n_in == 0)
        return AH_ERR_INVALID_ARG;
    if (reinterpret_cast<uintptr_t>(d_x) % 4 || reinterpret_cast<uintptr_t>(d_h_scales) % 8) return AH_ERR_INVALID_ARG;
    if (gate->n_out == 0) return AH_OK;
    if (gate->n_out > 0x7FFFFFE0u) return AH_ERR_INVALID_ARG;
    StreamParts sp = {};
    sp.n = 2;
    bool s0 = false, s1 = false;
    // whole units (not the latency launches' Q4_K pairs): each wave streams a few whole rows
    sp.p[0] = make_part(gate, src, d_x, d_scales, d_gate_y, nullptr, s0, false);
    sp.p[1] = make_part(up, src, d_x, d_scales, d_up_y, nullptr, s1, false);
    if (!s0 || !s1) return AH_ERR_INVALID_ARG;  // rows past one streaming tile
    const uint32_t kp = kpad_of(gate->n_in);
    AH_HIP(ctx, hipSetDevice(ctx->device));
    // hidden blocks per workgroup: as few as keep the grid resident (one round), at most kFfnMaxBlocks
    const uint32_t nb = (uint32_t)((gate->n_out + 31) / 32);
    const int occ = ah_ffn_occupancy(gate->type, kp);
    const uint64_t res = (uint64_t)(occ > 0 ? occ : 1) * (uint64_t)ctx->cu_count;
    uint32_t per = (uint32_t)((nb + res - 1) / res);
    per = per < 1 ? 1 : per > kFfnMaxBlocks ? kFfnMaxBlocks : per;
    FfnArgs fa = {d_h_codes, d_h_scales, (uint32_t)gate->n_out, per};
    AH_HIP(ctx, ah_launch_ffn_gate_up(gate->type, sp, fa, (nb + per - 1) / per, (uint32_t)ah_gemv_act_bytes(kp),
                                      ctx->d_status, pick(ctx, stream)));
    return AH_OK;
}

static int32_t ffn_launch(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const ah_tensor *down,
                          uint32_t src, const void *d_x, const int64_t *d_scales, float *d_y, int8_t *d_h_codes,
                          int64_t *d_h_scales, void *stream) {
    if (!ctx || !down || !d_y) return AH_ERR_INVALID_ARG;
    if (!gate || down->n_in != gate->n_out || down->n_out != gate->n_in) return AH_ERR_INVALID_ARG;
    if (reinterpret_cast<uintptr_t>(d_h_codes) % 4) return AH_ERR_INVALID_ARG;
    int32_t st = ffn_gate_up_launch(ctx, gate, up, src, d_x, d_scales, nullptr, nullptr, d_h_codes, d_h_scales, stream);
    if (st) return st;
    // the down projection's refusals go to the second status word (reported only when the
    // gate/up launch refused nothing)
    return gemv_launch(ctx, down, AH_SRC_CODES, d_h_codes, d_h_scales, d_y, nullptr, stream, ctx->d_status + 1);
}

int32_t ah_ffn_gate_up_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const float *d_x,
                           float *d_gate_y, float *d_up_y, int8_t *d_h_codes, int64_t *d_h_scales, void *stream) {
    return ffn_gate_up_launch(ctx, gate, up, AH_SRC_F32, d_x, nullptr, d_gate_y, d_up_y, d_h_codes, d_h_scales, stream);
}

int32_t ah_ffn_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const ah_tensor *down,
                   const float *d_x, float *d_y, int8_t *d_h_codes, int64_t *d_h_scales, void *stream) {
    return ffn_launch(ctx, gate, up, down, AH_SRC_F32, d_x, nullptr, d_y, d_h_codes, d_h_scales, stream);
}

int32_t ah_ffn_q8_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const ah_tensor *down,
                      const int8_t *d_codes, const int64_t *d_scales, float *d_y, int8_t *d_h_codes,
                      int64_t *d_h_scales, void *stream) {
    return ffn_launch(ctx, gate, up, down, AH_SRC_CODES, d_codes, d_scales, d_y, d_h_codes, d_h_scales, stream);
}

int32_t ah_swiglu_quant_dev(ah_ctx *ctx, const float *d_gate, const float *d_up, size_t n_tok, size_t n_ff,
                            int8_t *d_h_codes, int64_t *d_h_scales, void *stream) {
    if (!ctx) return AH_ERR_INVALID_ARG;
    if (n_tok == 0 || n_ff == 0) return AH_OK;
    if (!d_gate || !d_up || !d_h_codes || !d_h_scales) return AH_ERR_INVALID_ARG;
    if (reinterpret_cast<uintptr_t>(d_gate) % 4 || reinterpret_cast<uintptr_t>(d_up) % 4 ||
        reinterpret_cast<uintptr_t>(d_h_scales) % 8)
        return AH_ERR_INVALID_ARG;
    if (n_tok >= (1ull << 24) || n_ff >= (1ull << 31) || (uint64_t)n_tok * n_ff >= (1ull << 45)) return AH_ERR_INVALID_ARG;
    SwigluArgs a = {d_gate, d_up, d_h_codes, d_h_scales, (uint32_t)n_tok, (uint32_t)n_ff, 0ull,
                    (uint64_t)n_tok * n_ff, ctx->d_status};
    AH_HIP(ctx, hipSetDevice(ctx->device));
    AH_HIP(ctx, ah_launch_swiglu_quant(a, pick(ctx, stream)));
    return AH_OK;
}

int32_t ah_set_ffn_prefill_form(ah_ctx *ctx, uint32_t form) {
    if (!ctx || form > AH_FFN_PREFILL_TWO_PASS) return AH_ERR_INVALID_ARG;
    ctx->ffn_form = form;
    return AH_OK;
}

// The prefill FFN's gate/up (+ SwiGLU + hidden quantizer) from f32 x[n_tok][n_in] or, with
// src AH_SRC_CODES, a QuantAct per token (codes [n_tok][n_in], scales [n_tok][ceil(n_in/32)]).
static int32_t ffn_prefill_gate_up(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, uint32_t src,
                                   const void *d_x, const int64_t *d_scales, size_t n_tok, float *d_gate_y,
                                   float *d_up_y, int8_t *d_h_codes, int64_t *d_h_scales, void *stream) {
    if (!ctx || !gate || !up) return AH_ERR_INVALID_ARG;
    if (gate->type != up->type || gate->n_out != up->n_out || gate->n_in != up->n_in) return AH_ERR_INVALID_ARG;
    const size_t n_ff = gate->n_out;
    if (n_tok == 0 || n_ff == 0) return AH_OK;
    if (!d_x || !d_h_codes || !d_h_scales || gate->n_in == 0) return AH_ERR_INVALID_ARG;
    if (src == AH_SRC_CODES && !d_scales) return AH_ERR_INVALID_ARG;
    if ((src == AH_SRC_F32 && reinterpret_cast<uintptr_t>(d_x) % 4) || reinterpret_cast<uintptr_t>(d_h_scales) % 8 ||
        reinterpret_cast<uintptr_t>(d_gate_y) % 4 || reinterpret_cast<uintptr_t>(d_up_y) % 4)
        return AH_ERR_INVALID_ARG;
    // refusal keys up to 4 * n_tok * n_ff (gate, up, SwiGLU, hidden blocks)
    if (n_tok >= (1ull << 24) || (uint64_t)n_tok * n_ff >= (1ull << 45)) return AH_ERR_INVALID_ARG;
    const ah_tensor *w2[2] = {gate, up};
    const uint32_t t = gate->type;
    // AUTO takes the two passes: on MI355X at the configs[4] FFN (N = 512) they measured 110-139 us
    // against 175-197 us for the fused launch, whose SwiGLU epilogue runs at two waves per SIMD
    if (ctx->ffn_form == AH_FFN_PREFILL_FUSED && (t == AH_GGML_Q4_K || t == AH_GGML_Q2_K || t == AH_GGML_Q3_K)) {
        // one launch: gate and up rows of the same hidden indices in each tile, the SwiGLU and the
        // hidden quantizer in its epilogue
        GemmFfn f = {up->d, d_gate_y, d_up_y, d_h_codes, d_h_scales};
        float *y2[2] = {d_gate_y, d_up_y};
        GroupOpts o;
        o.ffn = &f;
        return gemm_group_launch(ctx, 2, w2, src, d_x, d_scales, n_tok, y2, stream, nullptr, 0, &o);
    }
    // two passes: gate and up as one grouped GEMM (part order: up's refusals keyed after all of
    // gate's), then
    // the SwiGLU + hidden quantizer over their f32 outputs
    float *g = d_gate_y, *u = d_up_y;
    if (!g || !u) {
        const size_t want = 2 * align256(n_tok * n_ff * 4);
        if (want > ctx->ffn_buf_bytes) {
            if (ctx->ffn_buf) {
                AH_HIP(ctx, hipDeviceSynchronize());  // queued kernels may still use the old buffer
                AH_HIP(ctx, hipFree(ctx->ffn_buf));
                ctx->ffn_buf = nullptr;
                ctx->ffn_buf_bytes = 0;
            }
            if (hipMalloc(&ctx->ffn_buf, want) != hipSuccess) {
                ctx->ffn_buf = nullptr;
                return AH_ERR_OUT_OF_MEMORY;
            }
            ctx->ffn_buf_bytes = want;
        }
        float *b = static_cast<float *>(ctx->ffn_buf);
        if (!g) g = b;
        if (!u) u = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(b) + align256(n_tok * n_ff * 4));
    }
    float *y2[2] = {g, u};
    int32_t st = gemm_group_launch(ctx, 2, w2, src, d_x, d_scales, n_tok, y2, stream);
    if (st) return st;
    const uint64_t NF = (uint64_t)n_tok * n_ff;
    SwigluArgs a = {g, u, d_h_codes, d_h_scales, (uint32_t)n_tok, (uint32_t)n_ff, 2 * NF, 3 * NF, ctx->d_status};
    AH_HIP(ctx, ah_launch_swiglu_quant(a, pick(ctx, stream)));
    return AH_OK;
}

int32_t ah_ffn_gate_up_prefill_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const float *d_x,
                                   size_t n_tok, float *d_gate_y, float *d_up_y, int8_t *d_h_codes,
                                   int64_t *d_h_scales, void *stream) {
    return ffn_prefill_gate_up(ctx, gate, up, AH_SRC_F32, d_x, nullptr, n_tok, d_gate_y, d_up_y, d_h_codes,
                               d_h_scales, stream);
}

static int32_t ffn_prefill(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const ah_tensor *down,
                           uint32_t src, const void *d_x, const int64_t *d_scales, size_t n_tok, float *d_y,
                           int8_t *d_h_codes, int64_t *d_h_scales, void *stream) {
    if (!ctx || !gate || !down) return AH_ERR_INVALID_ARG;
    if (down->n_in != gate->n_out || down->n_out != gate->n_in) return AH_ERR_INVALID_ARG;
    if (n_tok && down->n_out && !d_y) return AH_ERR_INVALID_ARG;
    if (reinterpret_cast<uintptr_t>(d_h_codes) % 4) return AH_ERR_INVALID_ARG;
    int32_t st = ffn_prefill_gate_up(ctx, gate, up, src, d_x, d_scales, n_tok, nullptr, nullptr, d_h_codes,
                                     d_h_scales, stream);
    if (st) return st;
    if (n_tok == 0 || down->n_out == 0) return AH_OK;
    // the down projection from the hidden QuantAct; its refusals go to the second status word
    // (reported only when nothing before it refused)
    GroupOpts o;
    o.status = ctx->d_status + 1;
    return gemm_group_launch(ctx, 1, &down, AH_SRC_CODES, d_h_codes, d_h_scales, n_tok, &d_y, stream, nullptr, 0,
                             &o);
}

int32_t ah_ffn_prefill_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const ah_tensor *down,
                           const float *d_x, size_t n_tok, float *d_y, int8_t *d_h_codes, int64_t *d_h_scales,
                           void *stream) {
    return ffn_prefill(ctx, gate, up, down, AH_SRC_F32, d_x, nullptr, n_tok, d_y, d_h_codes, d_h_scales, stream);
}

int32_t ah_ffn_prefill_q8_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const ah_tensor *down,
                              const int8_t *d_codes, const int64_t *d_scales, size_t n_tok, float *d_y,
                              int8_t *d_h_codes, int64_t *d_h_scales, void *stream) {
    return ffn_prefill(ctx, gate, up, down, AH_SRC_CODES, d_codes, d_scales, n_tok, d_y, d_h_codes, d_h_scales,
                       stream);
}

// ---- device buffers for callers without a HIP runtime of their own -----------------------------

int32_t ah_dev_alloc(ah_ctx *ctx, size_t bytes, void **d) {
    if (!ctx || !d) return AH_ERR_INVALID_ARG;
    *d = nullptr;
    if (bytes == 0) return AH_OK;
    AH_HIP(ctx, hipSetDevice(ctx->device));
    if (hipMalloc(d, bytes) != hipSuccess) {
        *d = nullptr;
        return AH_ERR_OUT_OF_MEMORY;
    }
    return AH_OK;
}

int32_t ah_dev_free(ah_ctx *ctx, void *d) {
    if (!ctx) return AH_ERR_INVALID_ARG;
    if (!d) return AH_OK;
    AH_HIP(ctx, hipSetDevice(ctx->device));
    AH_HIP(ctx, hipStreamSynchronize(ctx->stream));  // the context's queued work may still read it
    AH_HIP(ctx, hipFree(d));
    return AH_OK;
}

int32_t ah_copy_to_dev(ah_ctx *ctx, void *d_dst, const void *src, size_t bytes, void *stream) {
    if (!ctx || ((!d_dst || !src) && bytes)) return AH_ERR_INVALID_ARG;
    if (bytes == 0) return AH_OK;
    AH_HIP(ctx, hipSetDevice(ctx->device));
    AH_HIP(ctx, hipMemcpyAsync(d_dst, src, bytes, hipMemcpyHostToDevice, pick(ctx, stream)));
    // the host buffer may be reused as soon as the call returns
    AH_HIP(ctx, hipStreamSynchronize(pick(ctx, stream)));
    return AH_OK;
}

int32_t ah_copy_to_host(ah_ctx *ctx, void *dst, const void *d_src, size_t bytes, void *stream) {
    if (!ctx || ((!dst || !d_src) && bytes)) return AH_ERR_INVALID_ARG;
    if (bytes == 0) return AH_OK;
    AH_HIP(ctx, hipSetDevice(ctx->device));
    AH_HIP(ctx, hipMemcpyAsync(dst, d_src, bytes, hipMemcpyDeviceToHost, pick(ctx, stream)));
    AH_HIP(ctx, hipStreamSynchronize(pick(ctx, stream)));
    return AH_OK;
}

int32_t ah_gemv_plan_create(ah_ctx *ctx, size_t n_parts, const ah_tensor *const *w,
                            const float *const *d_x, float *const *d_y, ah_gemv_plan **out) {
    if (!ctx || !out || !w || !d_x || !d_y || n_parts == 0 || n_parts > 65536) return AH_ERR_INVALID_ARG;
    *out = nullptr;
    if (!w[0]) return AH_ERR_INVALID_ARG;
    GemvPart *parts = static_cast<GemvPart *>(std::calloc(n_parts, sizeof(GemvPart)));
    if (!parts) return AH_ERR_OUT_OF_MEMORY;
    uint32_t kpad_max = 0, nc = 4;
    bool all_stream = true, mixed = false;
    for (size_t i = 0; i < n_parts; ++i) {
        if (!w[i] || !d_x[i] || !d_y[i] || w[i]->n_out == 0 || reinterpret_cast<uintptr_t>(d_x[i]) % 4) {
            std::free(parts);
            return AH_ERR_INVALID_ARG;
        }
        mixed = mixed || w[i]->type != w[0]->type;
        bool st = false;
        parts[i] = make_part(w[i], AH_SRC_F32, d_x[i], nullptr, d_y[i], nullptr, st);
        parts[i].out_key0 = i ? parts[i - 1].out_key0 + w[i - 1]->n_out : 0;  // projection-then-row order
        all_stream = all_stream && st;
        const uint32_t kp = kpad_of(w[i]->n_in);
        kpad_max = kp > kpad_max ? kp : kpad_max;
        const uint32_t nci = ah_gemv_nc(parts[i].row_bytes);
        nc = nci > nc ? nci : nc;
    }
    // Parts of different GGUF types share one launch of the mixed-type streaming kernel, which
    // serves only parts whose rows fit its 8 KB wave tiles.
    if (mixed && !all_stream) {
        std::free(parts);
        return AH_ERR_INVALID_ARG;
    }
    const uint32_t type = mixed ? (uint32_t)kMixedType : w[0]->type;
    hipError_t e0 = hipSetDevice(ctx->device);
    if (e0 != hipSuccess) {
        std::free(parts);
        ctx->last_hip = (int)e0;
        return AH_ERR_HIP;
    }
    // A small streaming plan (every decode stage: q/k/v, o, gate/up, down, head) passes its parts
    // in the kernel arguments with whole workgroups per part, as a single projection does: a
    // workgroup then reaches its rows without the descriptor loads of the table plan, whose chain
    // (workgroup entry, then part, then activation) sits on the critical path of a stage that
    // streams one tile per wave.
    if (all_stream && n_parts <= kStreamArgParts) {
        ah_gemv_plan *p = new (std::nothrow) ah_gemv_plan();
        if (!p) {
            std::free(parts);
            return AH_ERR_OUT_OF_MEMORY;
        }
        const uint32_t wg = deal_wgs(parts, n_parts, resident_wgs(ctx, type, true, kpad_max), true);
        for (size_t i = 0; i < n_parts; ++i) p->sp.p[i] = parts[i];
        std::free(parts);
        if (wg == 0) {
            delete p;
            return AH_ERR_OUT_OF_MEMORY;
        }
        p->sp.n = (uint32_t)n_parts;
        p->type = type;
        p->n_parts = (uint32_t)n_parts;
        p->grid = wg;
        p->kpad_max = kpad_max;
        p->nc = nc;
        p->stream = true;
        p->arg_parts = true;
        p->act_bytes = (uint32_t)ah_gemv_act_bytes(kpad_max);
        *out = p;
        return AH_OK;
    }
    // A table plan serves many projections at once (throughput): its parts keep whole units.
    for (size_t i = 0; i < n_parts; ++i) {
        bool st = false;
        const uint64_t k0 = parts[i].out_key0;
        parts[i] = make_part(w[i], AH_SRC_F32, d_x[i], nullptr, d_y[i], nullptr, st, false);
        parts[i].out_key0 = k0;
    }
    // Streaming plan: waves dealt over the parts, activations sharing a workgroup's LDS region of
    // at most `budget` bytes (15 KB keeps two workgroups per CU; a larger activation raises it).
    if (all_stream) {
        size_t budget = 15360;
        for (size_t i = 0; i < n_parts; ++i) {
            const size_t a = ah_gemv_act_bytes(kpad_of(parts[i].n_in));
            budget = a > budget ? a : budget;
        }
        int occ = ah_gemv_stream_occupancy(type, budget + ah_gemv_stream_slot_bytes());
        if (occ < 1) occ = 1;
        const uint32_t n_res = (uint32_t)occ * (uint32_t)ctx->cu_count;
        StreamWG *wgd = static_cast<StreamWG *>(std::calloc(n_res, sizeof(StreamWG)));
        if (!wgd) {
            std::free(parts);
            return AH_ERR_OUT_OF_MEMORY;
        }
        const uint32_t nwg = deal_waves(parts, n_parts, n_res, budget, wgd);
        if (nwg) {
            ah_gemv_plan *p = new (std::nothrow) ah_gemv_plan();
            hipError_t e = p ? hipSuccess : hipErrorOutOfMemory;
            if (e == hipSuccess) e = hipMalloc(&p->d_parts, n_parts * sizeof(GemvPart));
            if (e == hipSuccess) e = hipMalloc(&p->d_wgd, (size_t)nwg * sizeof(StreamWG));
            if (e == hipSuccess) e = hipMemcpy(p->d_parts, parts, n_parts * sizeof(GemvPart), hipMemcpyHostToDevice);
            if (e == hipSuccess) e = hipMemcpy(p->d_wgd, wgd, (size_t)nwg * sizeof(StreamWG), hipMemcpyHostToDevice);
            std::free(parts);
            std::free(wgd);
            if (e != hipSuccess) {
                if (p) {
                    if (p->d_parts) (void)hipFree(p->d_parts);
                    if (p->d_wgd) (void)hipFree(p->d_wgd);
                    delete p;
                }
                ctx->last_hip = (int)e;
                return p ? AH_ERR_HIP : AH_ERR_OUT_OF_MEMORY;
            }
            p->type = type;
            p->n_parts = (uint32_t)n_parts;
            p->grid = nwg;
            p->kpad_max = kpad_max;
            p->nc = nc;
            p->stream = true;
            p->act_bytes = (uint32_t)budget;
            *out = p;
            return AH_OK;
        }
        std::free(wgd);
        if (mixed) {  // more parts than the resident waves: no single-type kernel can take them
            std::free(parts);
            return AH_ERR_INVALID_ARG;
        }
        all_stream = false;  // more parts than the resident waves: the workgroup-tile kernel
    }
    // one kernel serves the plan: every part as workgroup tiles
    for (size_t i = 0; i < n_parts; ++i) recut_wg_tiles(parts[i]);
    const uint32_t wg = deal_wgs(parts, n_parts, resident_wgs(ctx, type, all_stream, kpad_max), all_stream);
    if (wg == 0) {
        std::free(parts);
        return AH_ERR_OUT_OF_MEMORY;
    }
    uint32_t *map = static_cast<uint32_t *>(std::malloc((size_t)wg * sizeof(uint32_t)));
    if (!map) {
        std::free(parts);
        return AH_ERR_OUT_OF_MEMORY;
    }
    for (size_t i = 0; i < n_parts; ++i)
        for (uint32_t k = 0; k < parts[i].wg_count; ++k) map[parts[i].wg_begin + k] = (uint32_t)i;
    ah_gemv_plan *p = new (std::nothrow) ah_gemv_plan();
    if (!p) {
        std::free(parts);
        std::free(map);
        return AH_ERR_OUT_OF_MEMORY;
    }
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMalloc(&p->d_parts, n_parts * sizeof(GemvPart));
    if (e == hipSuccess) e = hipMalloc(&p->d_wg_part, (size_t)wg * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemcpy(p->d_parts, parts, n_parts * sizeof(GemvPart), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(p->d_wg_part, map, (size_t)wg * sizeof(uint32_t), hipMemcpyHostToDevice);
    std::free(parts);
    std::free(map);
    if (e != hipSuccess) {
        if (p->d_parts) (void)hipFree(p->d_parts);
        if (p->d_wg_part) (void)hipFree(p->d_wg_part);
        delete p;
        ctx->last_hip = (int)e;
        return AH_ERR_HIP;
    }
    p->type = type;
    p->n_parts = (uint32_t)n_parts;
    p->grid = wg;
    p->kpad_max = kpad_max;
    p->nc = nc;
    p->stream = all_stream;
    *out = p;
    return AH_OK;
}

int32_t ah_gemv_plan_run(ah_ctx *ctx, const ah_gemv_plan *plan, void *stream) {
    if (!ctx || !plan) return AH_ERR_INVALID_ARG;
    GemvPart none;
    std::memset(&none, 0, sizeof(none));
    AH_HIP(ctx, hipSetDevice(ctx->device));
    if (plan->arg_parts)
        AH_HIP(ctx, ah_launch_gemv_stream(plan->type, plan->sp, nullptr, nullptr, plan->grid,
                                          plan->act_bytes, ctx->d_status, pick(ctx, stream)));
    else if (plan->stream)
        AH_HIP(ctx, ah_launch_gemv_stream(plan->type, plan->sp, plan->d_parts, plan->d_wgd, plan->grid,
                                          plan->act_bytes, ctx->d_status, pick(ctx, stream)));
    else
        AH_HIP(ctx, ah_launch_gemv(plan->type, none, plan->d_parts, plan->d_wg_part, plan->grid,
                                   plan->kpad_max, plan->nc, ctx->d_status, pick(ctx, stream)));
    return AH_OK;
}

int32_t ah_gemv_plan_free(ah_ctx *ctx, ah_gemv_plan *plan) {
    if (!ctx || !plan) return AH_ERR_INVALID_ARG;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (plan->d_parts) (void)hipFree(plan->d_parts);
    if (plan->d_wg_part) (void)hipFree(plan->d_wg_part);
    if (plan->d_wgd) (void)hipFree(plan->d_wgd);
    delete plan;
    return AH_OK;
}

// ---- persistent decode sequence ----

static void seq_release(ah_seq *q) {
    if (!q) return;
    if (q->d_stages) (void)hipFree(q->d_stages);
    if (q->d_parts) (void)hipFree(q->d_parts);
    if (q->d_wgd) (void)hipFree(q->d_wgd);
    if (q->d_prod) (void)hipFree(q->d_prod);
    if (q->d_done) (void)hipFree(q->d_done);
    if (q->d_runs) (void)hipFree(q->d_runs);
    if (q->d_status) (void)hipFree(q->d_status);
    delete q;
}

int32_t ah_seq_create(ah_ctx *ctx, size_t n_stages, const ah_seq_stage *stages, ah_seq **out) {
    if (!ctx || !out || !stages || n_stages == 0 || n_stages > 65536) return AH_ERR_INVALID_ARG;
    *out = nullptr;
    // every GEMV part of every stage, stage by stage
    std::vector<GemvPart> parts;
    std::vector<size_t> first(n_stages, 0);
    uint32_t type = 0xFFFFFFFFu;
    bool mixed = false;
    size_t budget = 15360;
    for (size_t s = 0; s < n_stages; ++s) {
        const ah_seq_stage &S = stages[s];
        first[s] = parts.size();
        if (S.kind == AH_SEQ_SWIGLU) {
            if (!S.gate || !S.up || !S.h_codes || !S.h_scales || S.n == 0 || S.n > AH_MAX_N_IN ||
                reinterpret_cast<uintptr_t>(S.h_scales) % 8 || reinterpret_cast<uintptr_t>(S.h_codes) % 8)
                return AH_ERR_INVALID_ARG;
            continue;
        }
        if (S.kind != AH_SEQ_GEMV || S.n_parts == 0 || S.n_parts > 4096 || !S.w || !S.y) return AH_ERR_INVALID_ARG;
        for (size_t i = 0; i < S.n_parts; ++i) {
            const ah_tensor *w = S.w[i];
            const float *x = S.x ? S.x[i] : nullptr;
            const int8_t *c = S.codes ? S.codes[i] : nullptr;
            const int64_t *sc = S.scales ? S.scales[i] : nullptr;
            if (!w || w->n_out == 0 || !S.y[i]) return AH_ERR_INVALID_ARG;
            if (x ? reinterpret_cast<uintptr_t>(x) % 4 != 0
                  : (!c || !sc || reinterpret_cast<uintptr_t>(c) % 4 || reinterpret_cast<uintptr_t>(sc) % 8))
                return AH_ERR_INVALID_ARG;
            bool st = false;
            parts.push_back(make_part(w, x ? AH_SRC_F32 : AH_SRC_CODES, x ? static_cast<const void *>(x) : c,
                                      x ? nullptr : sc, S.y[i], nullptr, st));
            if (!st) return AH_ERR_INVALID_ARG;  // rows past the 8 KB streaming tile
            if (type != 0xFFFFFFFFu && type != w->type) mixed = true;
            type = w->type;
            const size_t a = ah_gemv_act_bytes(kpad_of(w->n_in));
            budget = a > budget ? a : budget;
        }
    }
    if (type == 0xFFFFFFFFu) type = AH_GGML_Q4_K;  // SwiGLU stages only
    if (mixed) type = kMixedType;
    AH_HIP(ctx, hipSetDevice(ctx->device));
    const int occ = ah_gemv_seq_occupancy(type, budget);
    if (occ < 1) return AH_ERR_INVALID_ARG;
    const uint32_t grid = (uint32_t)occ * (uint32_t)ctx->cu_count;
    if (grid > kSeqGroup * kSeqMaxGroups) return AH_ERR_INVALID_ARG;
    // one StreamWG table of `grid` entries per GEMV stage; workgroups past the dealt ones idle;
    // each stage's producers (workgroups with work) counted per group of kSeqGroup
    std::vector<SeqStage> dst(n_stages);
    std::vector<StreamWG> wgd;
    std::vector<uint32_t> prod(n_stages * kSeqMaxGroups, 0u);
    for (size_t s = 0; s < n_stages; ++s) {
        const ah_seq_stage &S = stages[s];
        SeqStage &D = dst[s];
        std::memset(&D, 0, sizeof(D));
        D.prod_off = (uint32_t)(s * kSeqMaxGroups);
        if (S.kind == AH_SEQ_SWIGLU) {
            const uint64_t nb = (S.n + 31) / 32;
            for (uint32_t g = 0; g < grid; ++g)
                if (nb * g / grid != nb * (g + 1) / grid) ++prod[s * kSeqMaxGroups + g / kSeqGroup];
            D.kind = kSeqSwiglu;
            D.n = (uint32_t)S.n;
            D.gate = S.gate;
            D.up = S.up;
            D.codes = S.h_codes;
            D.scales = S.h_scales;
            continue;
        }
        D.kind = kSeqGemv;
        D.wgd_off = (uint32_t)wgd.size();
        const size_t base = first[s];
        std::vector<StreamWG> tab(grid);
        const uint32_t nwg = deal_waves(parts.data() + base, S.n_parts, grid, budget, tab.data());
        if (nwg == 0) return AH_ERR_INVALID_ARG;
        for (uint32_t g = 0; g < grid; ++g) {
            StreamWG &T = tab[g];
            if (g >= nwg) {
                std::memset(&T, 0, sizeof(T));
                for (int v = 0; v < 8; ++v) T.wave_part[v] = kIdleWave;
            }
            if (T.n_act) ++prod[s * kSeqMaxGroups + g / kSeqGroup];
            for (int a = 0; a < 8; ++a) T.act_part[a] += (uint32_t)base;
            for (int v = 0; v < 8; ++v)
                if (T.wave_part[v] != kIdleWave) T.wave_part[v] += (uint32_t)base;
        }
        wgd.insert(wgd.end(), tab.begin(), tab.end());
    }
    ah_seq *q = new (std::nothrow) ah_seq();
    if (!q) return AH_ERR_OUT_OF_MEMORY;
    q->type = type;
    q->grid = grid;
    q->n_stages = (uint32_t)n_stages;
    q->act_bytes = (uint32_t)budget;
    std::vector<unsigned long long> none(n_stages, AH_ST_NONE);
    const size_t done_words = n_stages * kSeqMaxGroups * kSeqLine;
    hipError_t e = hipMalloc(&q->d_stages, n_stages * sizeof(SeqStage));
    if (e == hipSuccess && !parts.empty()) e = hipMalloc(&q->d_parts, parts.size() * sizeof(GemvPart));
    if (e == hipSuccess && !wgd.empty()) e = hipMalloc(&q->d_wgd, wgd.size() * sizeof(StreamWG));
    if (e == hipSuccess) e = hipMalloc(&q->d_prod, prod.size() * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&q->d_done, done_words * sizeof(unsigned));
    if (e == hipSuccess) e = hipMalloc(&q->d_runs, grid * sizeof(unsigned));
    if (e == hipSuccess) e = hipMalloc(&q->d_status, n_stages * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMemcpy(q->d_stages, dst.data(), n_stages * sizeof(SeqStage), hipMemcpyHostToDevice);
    if (e == hipSuccess && !parts.empty())
        e = hipMemcpy(q->d_parts, parts.data(), parts.size() * sizeof(GemvPart), hipMemcpyHostToDevice);
    if (e == hipSuccess && !wgd.empty())
        e = hipMemcpy(q->d_wgd, wgd.data(), wgd.size() * sizeof(StreamWG), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(q->d_prod, prod.data(), prod.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemset(q->d_done, 0, done_words * sizeof(unsigned));
    if (e == hipSuccess) e = hipMemset(q->d_runs, 0, grid * sizeof(unsigned));
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(q->d_status, none.data(), n_stages * sizeof(unsigned long long), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        seq_release(q);
        ctx->last_hip = (int)e;
        return AH_ERR_HIP;
    }
    *out = q;
    return AH_OK;
}

int32_t ah_seq_run(ah_ctx *ctx, const ah_seq *seq, void *stream) {
    if (!ctx || !seq) return AH_ERR_INVALID_ARG;
    SeqArgs a;
    a.stages = seq->d_stages;
    a.parts = seq->d_parts;
    a.wgd = seq->d_wgd;
    a.producers = seq->d_prod;
    a.done = seq->d_done;
    a.runs = seq->d_runs;
    a.status = seq->d_status;
    a.n_stages = seq->n_stages;
    a.act_bytes = seq->act_bytes;
    a.spin_limit = seq->spin_limit;
    AH_HIP(ctx, hipSetDevice(ctx->device));
    AH_HIP(ctx, ah_launch_gemv_seq(seq->type, a, seq->grid, pick(ctx, stream)));
    return AH_OK;
}

int32_t ah_seq_set_spin_limit(ah_seq *seq, uint32_t polls) {
    if (!seq) return AH_ERR_INVALID_ARG;
    seq->spin_limit = polls ? polls : kSeqSpinLimit;
    return AH_OK;
}

int32_t ah_seq_sync_status(ah_ctx *ctx, const ah_seq *seq, void *stream, uint32_t *stage) {
    if (!ctx || !seq) return AH_ERR_INVALID_ARG;
    AH_HIP(ctx, hipSetDevice(ctx->device));
    AH_HIP(ctx, hipStreamSynchronize(pick(ctx, stream)));
    std::vector<unsigned long long> st(seq->n_stages);
    AH_HIP(ctx, hipMemcpy(st.data(), seq->d_status, st.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost));
    for (uint32_t s = 0; s < seq->n_stages; ++s) {
        if (st[s] == AH_ST_NONE) continue;
        std::vector<unsigned long long> none(seq->n_stages, AH_ST_NONE);
        AH_HIP(ctx, hipMemcpy(seq->d_status, none.data(), none.size() * sizeof(unsigned long long), hipMemcpyHostToDevice));
        if (stage) *stage = s;
        return st[s] == kSeqTimeoutKey ? AH_ERR_SEQ_TIMEOUT : (int32_t)(st[s] & 0xffu);
    }
    return AH_OK;
}

int32_t ah_seq_info(const ah_seq *seq, uint32_t *grid, uint32_t *act_bytes) {
    if (!seq) return AH_ERR_INVALID_ARG;
    if (grid) *grid = seq->grid;
    if (act_bytes) *act_bytes = seq->act_bytes;
    return AH_OK;
}

int32_t ah_seq_free(ah_ctx *ctx, ah_seq *seq) {
    if (!ctx || !seq) return AH_ERR_INVALID_ARG;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    seq_release(seq);
    return AH_OK;
}

int32_t ah_gemm_f32_dev(ah_ctx *ctx, const ah_tensor *w, const float *d_x, size_t n_tok, float *d_y,
                        void *stream) {
    return gemm_launch(ctx, w, AH_SRC_F32, d_x, nullptr, n_tok, d_y, stream);
}

int32_t ah_gemm_f32_noalloc_dev(ah_ctx *ctx, const ah_tensor *w, const float *d_x, size_t n_tok,
                                float *d_y, void *stream) {
    if (!ctx || !w || !d_y || (!d_x && n_tok && w->n_in)) return AH_ERR_INVALID_ARG;
    if (n_tok == 0 || w->n_out == 0) return AH_OK;
    if (!ctx->noalloc) return AH_ERR_HIP;
    return gemm_group_launch(ctx, 1, &w, AH_SRC_F32, d_x, nullptr, n_tok, &d_y, stream, ctx->noalloc,
                             kNoAllocScratchBytes);
}

int32_t ah_set_gemm_design(ah_ctx *ctx, uint32_t ggml_type, uint32_t design) {
    if (!ctx || design > AH_GEMM_DESIGN_F16_TILE) return AH_ERR_INVALID_ARG;
    size_t qk = 0, bb = 0;
    if (!geom(ggml_type, qk, bb) || ggml_type >= 32) return AH_ERR_UNSUPPORTED_QUANT;
    if (design == AH_GEMM_DESIGN_INT8 && ggml_type != AH_GGML_Q8_0 && ggml_type != AH_GGML_Q4_K)
        return AH_ERR_UNSUPPORTED_QUANT;
    if (design == AH_GEMM_DESIGN_F16_TILE && ggml_type != AH_GGML_Q4_K && !ah_k23((int)ggml_type))
        return AH_ERR_UNSUPPORTED_QUANT;
    ctx->design[ggml_type] = design;
    return AH_OK;
}

int32_t ah_ctx_scratch_bytes(const ah_ctx *ctx, size_t *bytes) {
    if (!ctx || !bytes) return AH_ERR_INVALID_ARG;
    *bytes = ctx->scratch_bytes;
    return AH_OK;
}

int32_t ah_gemm_noalloc_scratch_bytes(size_t *bytes) {
    if (!bytes) return AH_ERR_INVALID_ARG;
    *bytes = kNoAllocScratchBytes;
    return AH_OK;
}

int32_t ah_gemm_q8_dev(ah_ctx *ctx, const ah_tensor *w, const int8_t *d_codes, const int64_t *d_scales,
                       size_t n_tok, float *d_y, void *stream) {
    if (!d_scales && n_tok) return AH_ERR_INVALID_ARG;
    return gemm_launch(ctx, w, AH_SRC_CODES, d_codes, d_scales, n_tok, d_y, stream);
}

int32_t ah_gemm_group_f32_dev(ah_ctx *ctx, size_t n_parts, const ah_tensor *const *w, const float *d_x,
                              size_t n_tok, float *const *d_y, void *stream) {
    return gemm_group_launch(ctx, n_parts, w, AH_SRC_F32, d_x, nullptr, n_tok, d_y, stream);
}

int32_t ah_gemm_group_q8_dev(ah_ctx *ctx, size_t n_parts, const ah_tensor *const *w, const int8_t *d_codes,
                             const int64_t *d_scales, size_t n_tok, float *const *d_y, void *stream) {
    if (!d_scales && n_tok) return AH_ERR_INVALID_ARG;
    return gemm_group_launch(ctx, n_parts, w, AH_SRC_CODES, d_codes, d_scales, n_tok, d_y, stream);
}

int32_t ah_sync_status(ah_ctx *ctx, void *stream) {
    if (!ctx) return AH_ERR_INVALID_ARG;
    AH_HIP(ctx, hipSetDevice(ctx->device));
    AH_HIP(ctx, hipStreamSynchronize(pick(ctx, stream)));
    unsigned long long keys[2] = {AH_ST_NONE, AH_ST_NONE};
    AH_HIP(ctx, hipMemcpy(keys, ctx->d_status, sizeof(keys), hipMemcpyDeviceToHost));
    if (keys[0] == AH_ST_NONE && keys[1] == AH_ST_NONE) return AH_OK;
    int32_t r = reset_status(ctx);
    if (r) return r;
    return (int32_t)((keys[0] != AH_ST_NONE ? keys[0] : keys[1]) & 0xffu);
}

// ---- diagnostics ----

int32_t ah_probe_mfma_peak(ah_ctx *ctx, uint32_t kind, double *tera_ops) {
    if (!ctx || !tera_ops || kind > 1) return AH_ERR_INVALID_ARG;
    const size_t o_sink = 256, sink_bytes = (size_t)2 * ctx->cu_count * 256 * 4;
    int32_t st = ensure_scratch(ctx, o_sink + sink_bytes);
    if (st) return st;
    uint8_t *S = static_cast<uint8_t *>(ctx->scratch);
    const uint32_t seed[8] = {0x9e3779b9u, 0x7f4a7c15u, 0x85ebca6bu, 0xc2b2ae35u,
                              0x27d4eb2fu, 0x165667b1u, 0xd3a2646cu, 0xfd7046c5u};
    AH_HIP(ctx, hipSetDevice(ctx->device));
    AH_HIP(ctx, hipMemcpy(S, seed, sizeof(seed), hipMemcpyHostToDevice));
    AH_HIP(ctx, ah_probe_mfma(kind, (uint32_t)ctx->cu_count, reinterpret_cast<const uint32_t *>(S),
                              reinterpret_cast<uint32_t *>(S + o_sink), ctx->stream, tera_ops));
    return AH_OK;
}

// ---- host convenience forms ----

int32_t ah_matvec_q8act(ah_ctx *ctx, const ah_tensor *w, const int8_t *codes, const int64_t *scales,
                        size_t n_codes, float *y) {
    if (!ctx || !w || (!y && w->n_out)) return AH_ERR_INVALID_ARG;
    if (n_codes != w->n_in) return AH_ERR_SHAPE_MISMATCH;
    const size_t nb = (w->n_in + 31) / 32;
    const size_t oc = 0, os = align256(w->n_in), oy = align256(os + nb * 8);
    int32_t st = ensure_scratch(ctx, oy + w->n_out * 4);
    if (st) return st;
    uint8_t *S = static_cast<uint8_t *>(ctx->scratch);
    AH_HIP(ctx, hipSetDevice(ctx->device));
    if (w->n_in) {
        AH_HIP(ctx, hipMemcpy(S + oc, codes, w->n_in, hipMemcpyHostToDevice));
        AH_HIP(ctx, hipMemcpy(S + os, scales, nb * 8, hipMemcpyHostToDevice));
    }
    st = gemv_launch(ctx, w, AH_SRC_CODES, S + oc, reinterpret_cast<int64_t *>(S + os),
                     reinterpret_cast<float *>(S + oy), nullptr, nullptr);
    if (st) return st;
    st = ah_sync_status(ctx, nullptr);
    if (st) return st;
    if (w->n_out) AH_HIP(ctx, hipMemcpy(y, S + oy, w->n_out * 4, hipMemcpyDeviceToHost));
    return AH_OK;
}

int32_t ah_matmat_q8act(ah_ctx *ctx, const ah_tensor *w, const int8_t *codes, const int64_t *scales,
                        size_t n_tok, float *y) {
    if (!ctx || !w || (!y && n_tok && w->n_out)) return AH_ERR_INVALID_ARG;
    if (n_tok == 0 || w->n_out == 0) return AH_OK;
    const size_t nb = (w->n_in + 31) / 32;
    // inputs live in a separate allocation: gemm_launch grows ctx->scratch for its operands
    const size_t in_bytes = align256(n_tok * w->n_in) + align256(n_tok * nb * 8) + n_tok * w->n_out * 4;
    uint8_t *buf = nullptr;
    AH_HIP(ctx, hipSetDevice(ctx->device));
    if (hipMalloc(&buf, in_bytes) != hipSuccess) return AH_ERR_OUT_OF_MEMORY;
    int8_t *dc = reinterpret_cast<int8_t *>(buf);
    int64_t *ds = reinterpret_cast<int64_t *>(buf + align256(n_tok * w->n_in));
    float *dy = reinterpret_cast<float *>(buf + align256(n_tok * w->n_in) + align256(n_tok * nb * 8));
    hipError_t e = hipSuccess;
    if (w->n_in) {
        e = hipMemcpy(dc, codes, n_tok * w->n_in, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(ds, scales, n_tok * nb * 8, hipMemcpyHostToDevice);
    }
    int32_t st = e == hipSuccess ? gemm_launch(ctx, w, AH_SRC_CODES, dc, ds, n_tok, dy, nullptr) : AH_ERR_HIP;
    if (st == AH_OK) st = ah_sync_status(ctx, nullptr);
    if (st == AH_OK && hipMemcpy(y, dy, n_tok * w->n_out * 4, hipMemcpyDeviceToHost) != hipSuccess) st = AH_ERR_HIP;
    (void)hipFree(buf);
    if (e != hipSuccess) ctx->last_hip = (int)e;
    return st;
}

int32_t ah_quant_act(ah_ctx *ctx, const int64_t *x, size_t n, int8_t *codes, int64_t *scales) {
    if (!ctx || ((!x || !codes || !scales) && n)) return AH_ERR_INVALID_ARG;
    if (n == 0) return AH_OK;
    const size_t nb = (n + 31) / 32;
    const size_t ox = 0, oc = align256(n * 8), os = align256(oc + n);
    int32_t st = ensure_scratch(ctx, os + nb * 8);
    if (st) return st;
    uint8_t *S = static_cast<uint8_t *>(ctx->scratch);
    AH_HIP(ctx, hipSetDevice(ctx->device));
    AH_HIP(ctx, hipMemcpy(S + ox, x, n * 8, hipMemcpyHostToDevice));
    st = quant_dev(ctx, AH_SRC_Q32, S + ox, 1, n, reinterpret_cast<int8_t *>(S + oc),
                   reinterpret_cast<int64_t *>(S + os), nullptr);
    if (st) return st;
    st = ah_sync_status(ctx, nullptr);
    if (st) return st;
    AH_HIP(ctx, hipMemcpy(codes, S + oc, n, hipMemcpyDeviceToHost));
    AH_HIP(ctx, hipMemcpy(scales, S + os, nb * 8, hipMemcpyDeviceToHost));
    return AH_OK;
}

}  // extern "C"
