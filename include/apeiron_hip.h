/*
 * apeiron_hip.h -- C ABI of the MI355X (gfx950) backend for apeiron's quantized
 * linear-layer path: GGUF block-quantized weights (Q8_0, Q5_0, Q2_K, Q3_K, Q4_K, Q6_K) times the
 * power-of-two int8 activation quantizer, as a GEMV at decode (N = 1) and a GEMM at
 * prefill (N > 1).
 *
 * Every function is extern "C", takes plain pointers and sizes, and returns an int32
 * status.  No exceptions cross the ABI.  All paths cited below are in the apeiron tree.
 *
 * Conventions
 *   - Weights live on the device in their GGUF block layout: n_out rows of ceil(n_in/qk) whole
 *     blocks (ops/matvec.rs:164-175).  One exception, made by ah_upload_weight only: a Q4_K row
 *     whose n_in is not a multiple of 256 (n_in <= 8192) is stored without the trailing qs
 *     chunks of its last super-block, which the product never reads (ah_tensor_info reports the
 *     device row stride).  Results are identical either way.
 *   - Activations are f32 (converted exactly as F32::to_q32, num/fp.rs:186-230) or
 *     Q32.32 int64 (the engine's own type, engine/mod.rs:58-80), or already quantized
 *     (codes int8 + scales int64, the QuantAct of chart/mod.rs:67-81).
 *   - Outputs are f32 real values.  The reference's Q32.32 value of row o is
 *     round_shift_32(sum_i w_oi * xhat_i); the f32 output is that sum * 2^-32 computed
 *     from exact per-group integer dots with f32 accumulation.
 *   - Functions suffixed _dev take DEVICE pointers and enqueue on `stream`
 *     (a hipStream_t; NULL = the context's own stream); they return once enqueued.
 *     Data-dependent refusals (non-finite or out-of-range input, an activation with no
 *     Q32.32 value) are recorded on the device and returned by ah_sync_status().
 *   - Functions without the suffix take HOST pointers and are synchronous.
 *   - A context is not thread-safe; callers serialise on it (as the reference's pool lock,
 *     chart/pool.rs:496-505).
 */
#ifndef APEIRON_HIP_H
#define APEIRON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: one per MatvecError variant (ops/matvec.rs:11-48) + boundary codes ---- */
#define AH_OK 0
#define AH_ERR_SHAPE_MISMATCH 1       /* MatvecError::ShapeMismatch                       */
#define AH_ERR_ROW_LENGTH 2           /* MatvecError::RowLength                           */
#define AH_ERR_SHORT_PAYLOAD 3        /* MatvecError::ShortPayload                        */
#define AH_ERR_LENGTH_OVERFLOW 4      /* MatvecError::LengthOverflow                      */
#define AH_ERR_UNSUPPORTED_QUANT 5    /* MatvecError::UnsupportedQuant                    */
#define AH_ERR_NONFINITE_SCALE 6      /* MatvecError::Dequant(EngineError::NonFiniteScale)*/
#define AH_ERR_FIXED_OVERFLOW 7       /* MatvecError::Dequant(EngineError::FixedOverflow) */
#define AH_ERR_ACCUMULATOR_OVERFLOW 8 /* MatvecError::AccumulatorOverflow                 */
#define AH_ERR_OUTPUT_OVERFLOW 9      /* MatvecError::OutputOverflow                      */
#define AH_ERR_NONFINITE_INPUT 10     /* F32Error::NonFinite (num/f32_convert.rs:44-49)   */
#define AH_ERR_INPUT_RANGE 11         /* F32Error::OutOfRange                             */
#define AH_ERR_FFN_OVERFLOW 12        /* FfnError::Overflow (ops/ffn.rs:11-27)            */
#define AH_ERR_EXP_RANGE 13           /* FfnError::ExpOutOfRange                          */
#define AH_ERR_ZERO_DENOMINATOR 14    /* FfnError::ZeroDenominator                        */
#define AH_ERR_NO_DEVICE 20           /* no usable gfx950 device (the honest skip of       */
                                      /* Vk::load, gpu/vulkan.rs:1097-1106)               */
#define AH_ERR_INVALID_ARG 21         /* null pointer / bad handle / limits exceeded       */
#define AH_ERR_HIP 22                 /* a HIP runtime call failed                         */
#define AH_ERR_OUT_OF_MEMORY 23
#define AH_ERR_SCRATCH_LIMIT 24       /* a no-alloc call needs more than its fixed scratch  */
#define AH_ERR_SEQ_TIMEOUT 25         /* a sequence's grid barrier waited past its limit    */

/* ggml type ids (format/quant.rs:20-49) */
#define AH_GGML_Q5_0 6   /* format/quant.rs:28-29, :261-297 */
#define AH_GGML_Q8_0 8
#define AH_GGML_Q2_K 10  /* format/quant.rs:30-31, :308-386; GEMM: one GEMV launch per token */
#define AH_GGML_Q3_K 11  /* format/quant.rs:32-33, :388-476; GEMM: one GEMV launch per token */
#define AH_GGML_Q4_K 12
#define AH_GGML_Q6_K 14

/* Largest n_in the GEMV keeps in LDS and the GEMM stages (both kernels refuse beyond). */
#define AH_MAX_N_IN 32768

typedef struct ah_ctx ah_ctx;
typedef struct ah_tensor ah_tensor;

/* ---- lifecycle ---------------------------------------------------------------------------- */

/* Open device `device`, create the context stream.  AH_ERR_NO_DEVICE when there is no GPU
 * or it is not gfx950.  (Boundary analogue of Vk::load, gpu/vulkan.rs:1097-1106.) */
int32_t ah_init(int32_t device, ah_ctx **out);
int32_t ah_destroy(ah_ctx *ctx);
/* Human-readable name of a status code (static string). */
const char *ah_status_str(int32_t status);
/* The last HIP error the context saw (hipError_t as int), for diagnostics. */
int32_t ah_last_hip_error(const ah_ctx *ctx);
/* The f16 bit pattern of the first non-finite block scale (row order; d before dmin) behind the
 * context's most recent AH_ERR_NONFINITE_SCALE: the `bits` of the reference's
 * EngineError::NonFiniteScale { bits } (num/dequant.rs:25-41). */
int32_t ah_last_refusal_bits(const ah_ctx *ctx, uint32_t *bits);

/* ---- weights -------------------------------------------------------------------------------- */

/* Copy an n_out x n_in GGUF payload (host bytes) to the device (ragged Q4_K rows compacted, see
 * Conventions).
 * Validates geometry like matvec_fixed (ops/matvec.rs:160-175: UNSUPPORTED_QUANT,
 * LENGTH_OVERFLOW, SHORT_PAYLOAD) and scans every f16 block scale (d, dmin) for Inf/NaN:
 * a non-finite tensor is refused with AH_ERR_NONFINITE_SCALE, the refusal the reference's
 * row dequantizer makes for it (num/dequant.rs:25-41), so the caller keeps its CPU path.
 * Replaces the resident-GGUF borrow of the reference (loader.rs:421-434, step.rs:375). */
int32_t ah_upload_weight(ah_ctx *ctx, uint32_t ggml_type, const void *raw, size_t raw_len,
                         size_t n_out, size_t n_in, ah_tensor **out);
/* Wrap a payload already in device memory (not copied, not owned; must outlive the tensor).
 * The f16 scale scan runs on the device. */
int32_t ah_wrap_weight_dev(ah_ctx *ctx, uint32_t ggml_type, const void *d_raw, size_t raw_len,
                           size_t n_out, size_t n_in, ah_tensor **out);
int32_t ah_free_tensor(ah_ctx *ctx, ah_tensor *t);
/* Geometry of a tensor: ggml type, n_out, n_in, device row stride in bytes, device pointer. */
int32_t ah_tensor_info(const ah_tensor *t, uint32_t *ggml_type, size_t *n_out, size_t *n_in,
                       size_t *row_bytes, const void **d_raw);

/* ---- activation quantizer (chart/mod.rs:258 quant_act; chart/ffn.rs:130,200 pooled forms) ---- */

/* n_tok rows of n_in activations -> codes[n_tok][n_in] int8 and scales[n_tok][ceil(n_in/32)]
 * int64 (Q32.32 power-of-two scales), bit-exact to quant_act(to_q32(x)) per row. */
int32_t ah_quant_act_f32_dev(ah_ctx *ctx, const float *d_x, size_t n_tok, size_t n_in,
                             int8_t *d_codes, int64_t *d_scales, void *stream);
/* Same from Q32.32 int64 activations (the engine's native Vec<i64>). */
int32_t ah_quant_act_q32_dev(ah_ctx *ctx, const int64_t *d_x, size_t n_tok, size_t n_in,
                             int8_t *d_codes, int64_t *d_scales, void *stream);

/* ---- decode GEMV, N = 1 (chart/mod.rs:1887 matvec_q8act; chart/ffn.rs:667 chunked form) ---- */

/* y[n_out] = W x with the quantizer fused into the kernel prologue. */
int32_t ah_gemv_f32_dev(ah_ctx *ctx, const ah_tensor *w, const float *d_x, float *d_y,
                        void *stream);
/* y[n_out] = W x from pre-quantized codes[n_in] + scales[ceil(n_in/32)].  d_codes must be
 * 4-byte aligned (the kernel reads codes a dword at a time; AH_ERR_INVALID_ARG otherwise). */
int32_t ah_gemv_q8_dev(ah_ctx *ctx, const ah_tensor *w, const int8_t *d_codes,
                       const int64_t *d_scales, float *d_y, void *stream);

/* Grouped GEMV: n_parts independent projections in ONE launch, each with its own weight,
 * f32 input and output (chart/ffn.rs:925 projections_q8act shares one dispatch for q/k/v;
 * here every part may have its own input).  Parts may mix ggml types (a Q4_K_M model's Q4_K and
 * Q6_K projections in one launch) when every part's rows fit the streaming kernel's 8 KB tiles
 * (Q8_0 K <= 7680, Q4_K K <= 14336, Q6_K K <= 9728); otherwise a mixed plan is refused with
 * AH_ERR_INVALID_ARG and a single-type plan falls back to the workgroup-tile kernel.  A plan fixes
 * the device pointers once (descriptors and the waves' assignment, dealt over the parts by tiles,
 * are uploaded at creation), so running it is one launch
 * with no host-device traffic -- the form a per-token projection sequence replays. */
typedef struct ah_gemv_plan ah_gemv_plan;
int32_t ah_gemv_plan_create(ah_ctx *ctx, size_t n_parts, const ah_tensor *const *w,
                            const float *const *d_x, float *const *d_y, ah_gemv_plan **out);
int32_t ah_gemv_plan_run(ah_ctx *ctx, const ah_gemv_plan *plan, void *stream);
int32_t ah_gemv_plan_free(ah_ctx *ctx, ah_gemv_plan *plan);

/* Fused FFN (ffn_q8act_prepared_into, chart/ffn.rs:1609; fused_ffn_task, chart/ffn.rs:1532-1594):
 * h = quant_act(round_shift_32(silu_fixed(to_q32(gate . x)) * to_q32(up . x))) exactly
 * (ops/ffn.rs:80, ops/silu.rs:18-60, chart/ffn.rs:246-252), then y = down . h.
 * ah_ffn_gate_up_dev is ONE launch: gate and up rows stream in the same workgroups (waves 0-3
 * gate, 4-7 up, over 32-row hidden blocks), their row sums meet in LDS and the workgroup's
 * epilogue writes the hidden QuantAct: d_h_codes[n_ff] (int8) and d_h_scales[ceil(n_ff/32)]
 * (int64; 8-byte aligned).  gate and up share type and shape (n_ff x n_embd) and take the same
 * f32 input d_x[n_embd] (4-byte aligned); d_gate_y / d_up_y (optional, NULL to skip) receive
 * the f32 gate and up values the SwiGLU consumed.  Their rows must fit the streaming kernel's
 * 8 KB tiles (Q8_0 K <= 7680, Q4_K K <= 14336, Q6_K K <= 9728), else AH_ERR_INVALID_ARG.
 * ah_ffn_dev adds the down projection (n_embd x n_ff, any type) from that QuantAct (d_h_codes
 * 4-byte aligned): two launches.  Refusals (ah_sync_status) in the reference FFN's order
 * (chart/ffn.rs:1712-1720): the input's conversion and quantization, gate then up outputs, the
 * hidden elements' conversion or SwiGLU (AH_ERR_FFN_OVERFLOW, AH_ERR_EXP_RANGE,
 * AH_ERR_ZERO_DENOMINATOR), the hidden quantizer's, and only when none of those occurred, the
 * down projection's. */
int32_t ah_ffn_gate_up_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const float *d_x,
                           float *d_gate_y, float *d_up_y, int8_t *d_h_codes, int64_t *d_h_scales,
                           void *stream);
int32_t ah_ffn_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const ah_tensor *down,
                   const float *d_x, float *d_y, int8_t *d_h_codes, int64_t *d_h_scales, void *stream);
/* ah_ffn_dev from a QuantAct (the engine's own quantized activation, ffn_q8act_prepared_into's
 * `q = quantize(x)`): d_codes[n_embd] (4-byte aligned) and d_scales[ceil(n_embd/32)] (8-byte
 * aligned) in place of the f32 input; the same launches and refusal order after the input's. */
int32_t ah_ffn_q8_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const ah_tensor *down,
                      const int8_t *d_codes, const int64_t *d_scales, float *d_y, int8_t *d_h_codes,
                      int64_t *d_h_scales, void *stream);

/* Prefill FFN, N = n_tok > 1 (the step's column path, step/cols.rs:1026-1067: quant_cols, the
 * [W_gate; W_up] GEMM with the SwiGLU epilogue, gemm_q8_0_swiglu_carrier, kern/gemm.rs:955-1168,
 * or gate/up proj_cols + swiglu_cols, chart/ffn.rs:493-560; then the down proj_cols).  For every
 * token t and hidden index i: h[t][i] = round_shift_32(silu_fixed(to_q32(gate[t][i])) *
 * to_q32(up[t][i])) exactly, from the f32 gate / up values of the GEMM (within the GEMM's
 * tolerance of the exact projections), and the hidden QuantAct: d_h_codes[n_tok][n_ff] (int8)
 * and d_h_scales[n_tok][ceil(n_ff/32)] (int64, 8-byte aligned), quant_act of each token's row.
 * ah_ffn_gate_up_prefill_dev takes f32 input d_x[n_tok][n_embd]; d_gate_y / d_up_y (optional,
 * [n_tok][n_ff], NULL to skip) receive the f32 gate and up values the SwiGLU consumed.  Q4_K,
 * Q2_K and Q3_K run as ONE launch (after the input's operand pass): the dequantize-once tiles
 * hold gate and up rows of the same 64 hidden indices, and the epilogue writes the hidden
 * QuantAct (no gate / up matrix in memory) -- the form ah_set_ffn_prefill_form selects with
 * AH_FFN_PREFILL_FUSED; the default (AUTO, and every other type) runs the grouped gate/up GEMM,
 * then a SwiGLU pass (ah_swiglu_quant_dev's kernel), which measured faster on MI355X.
 * ah_ffn_prefill_dev adds the down projection (n_embd x n_ff, any type) from the hidden QuantAct
 * (d_h_codes 4-byte aligned) into d_y[n_tok][n_embd].  Refusals (ah_sync_status) in the
 * reference FFN's order: the input's quantization, the gate projection's outputs (token-major),
 * then the up projection's, the elements' conversion or SwiGLU (AH_ERR_FFN_OVERFLOW,
 * AH_ERR_EXP_RANGE, AH_ERR_ZERO_DENOMINATOR; token-major), the hidden quantizer's, and only when
 * none of those occurred, the down projection's.  Uses the context's GEMM scratch (as
 * ah_gemm_f32_dev) and, for the two-pass form without d_gate_y / d_up_y, a context buffer of
 * 8 * n_tok * n_ff bytes (grown on demand). */
int32_t ah_ffn_gate_up_prefill_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const float *d_x,
                                   size_t n_tok, float *d_gate_y, float *d_up_y, int8_t *d_h_codes,
                                   int64_t *d_h_scales, void *stream);
int32_t ah_ffn_prefill_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const ah_tensor *down,
                           const float *d_x, size_t n_tok, float *d_y, int8_t *d_h_codes, int64_t *d_h_scales,
                           void *stream);
/* ah_ffn_prefill_dev from the columns' QuantActs (step/cols.rs:1026's `qs = quant_cols(xs)`):
 * d_codes[n_tok][n_embd] and d_scales[n_tok][ceil(n_embd/32)] (8-byte aligned). */
int32_t ah_ffn_prefill_q8_dev(ah_ctx *ctx, const ah_tensor *gate, const ah_tensor *up, const ah_tensor *down,
                              const int8_t *d_codes, const int64_t *d_scales, size_t n_tok, float *d_y,
                              int8_t *d_h_codes, int64_t *d_h_scales, void *stream);
/* The prefill FFN's form per context: AUTO (the default: two passes), FUSED (one launch for
 * Q4_K / Q2_K / Q3_K gate/up; other types keep two passes) or TWO_PASS.  The hidden QuantAct is
 * bit-identical given the same gate / up values; those agree within the GEMM tolerance. */
#define AH_FFN_PREFILL_AUTO 0u
#define AH_FFN_PREFILL_FUSED 1u
#define AH_FFN_PREFILL_TWO_PASS 2u
int32_t ah_set_ffn_prefill_form(ah_ctx *ctx, uint32_t form);
/* swiglu_cols + quant_cols (chart/ffn.rs:493-560, chart/mod.rs:258-334) over f32 gate / up
 * values [n_tok][n_ff] (4-byte aligned): the hidden QuantAct as above.  Refusals token-major: an
 * element's conversion or SwiGLU, then the quantizer's blocks. */
int32_t ah_swiglu_quant_dev(ah_ctx *ctx, const float *d_gate, const float *d_up, size_t n_tok, size_t n_ff,
                            int8_t *d_h_codes, int64_t *d_h_scales, void *stream);

/* Device buffers and copies for callers that bind only this library (no HIP runtime of their
 * own, as the engine's dlopen binding): the device-pointer forms above take these.  No
 * counterpart in the reference (its CPU path owns host memory only; its Vulkan backend allocates
 * through its own device object).  ah_dev_free first waits for the context's stream.  The copies
 * run on `stream` (NULL: the context's) and return once complete, so the host buffer may be
 * reused at once. */
int32_t ah_dev_alloc(ah_ctx *ctx, size_t bytes, void **d);
int32_t ah_dev_free(ah_ctx *ctx, void *d);
int32_t ah_copy_to_dev(ah_ctx *ctx, void *d_dst, const void *src, size_t bytes, void *stream);
int32_t ah_copy_to_host(ah_ctx *ctx, void *dst, const void *d_src, size_t bytes, void *stream);

/* Persistent decode sequence: a token's chain of projection stages in ONE launch.  Stage s may
 * read outputs of stages before it (q/k/v -> o -> gate/up -> SwiGLU -> down per layer, then the
 * head): every workgroup of a resident grid finishes its share of stage s, then all meet at a
 * grid barrier before stage s+1 reads its inputs; each wave requests its first stage-(s+1) weight
 * tile before it waits, so the weight stream runs on through the barriers.  Replaces the
 * engine's per-projection dispatches of a decode step (projections_q8act, chart/ffn.rs:905-1098;
 * Vulkan's one command buffer per token, gpu/decode/model.rs:1-12).  A SwiGLU stage is the
 * reference's fused FFN step (fused_ffn_task, chart/ffn.rs:1532-1594): for each hidden index
 * h = round_shift_32(silu_fixed(to_q32(gate)) * to_q32(up)) exactly (ops/silu.rs:18-60,
 * chart/ffn.rs:246-252), quantized (quant_act) into a QuantAct that a later GEMV stage takes as
 * pre-quantized input, so gate/up -> SwiGLU -> down runs without leaving the launch.
 * Limits: every GEMV part's rows fit the streaming kernel's 8 KB tiles (Q8_0 K <= 7680, Q4_K
 * K <= 14336, Q6_K K <= 9728), at most 8 parts per stage per workgroup's activation budget
 * (as ah_gemv_plan_create), at most 65536 stages. */
#define AH_SEQ_GEMV 0
#define AH_SEQ_SWIGLU 1
typedef struct ah_seq ah_seq;
typedef struct ah_seq_stage {
    uint32_t kind;                 /* AH_SEQ_GEMV or AH_SEQ_SWIGLU */
    /* AH_SEQ_GEMV: n_parts projections, each from an f32 input x[i] or, when x[i] is NULL, from a
     * QuantAct codes[i] / scales[i] (e.g. a SwiGLU stage's output; codes 4-byte aligned) */
    size_t n_parts;
    const ah_tensor *const *w;
    const float *const *x;
    const int8_t *const *codes;    /* may be NULL when every x[i] is given */
    const int64_t *const *scales;
    float *const *y;
    /* AH_SEQ_SWIGLU: n hidden values from f32 gate[n] / up[n] into h_codes[n] / h_scales[ceil(n/32)] */
    const float *gate;
    const float *up;
    size_t n;
    int8_t *h_codes;
    int64_t *h_scales;
} ah_seq_stage;
/* Plans the sequence (every device pointer is fixed here) and uploads its tables. */
int32_t ah_seq_create(ah_ctx *ctx, size_t n_stages, const ah_seq_stage *stages, ah_seq **out);
/* Enqueues the whole sequence as one launch on `stream`; its grid is what the device holds at
 * once, so the stages' grid barriers need the device to itself for the run (other work holding
 * CUs delays some workgroups: the bounded waits then give up and the run reports
 * AH_ERR_SEQ_TIMEOUT). */
int32_t ah_seq_run(ah_ctx *ctx, const ah_seq *seq, void *stream);
/* Synchronizes `stream`, then returns (and clears) the first refusal of the sequence's last runs
 * in stage order, as ah_sync_status does per call; *stage (optional) receives its stage index.
 * AH_ERR_SEQ_TIMEOUT: a grid barrier waited past its limit (the run's outputs are not valid). */
int32_t ah_seq_sync_status(ah_ctx *ctx, const ah_seq *seq, void *stream, uint32_t *stage);
int32_t ah_seq_free(ah_ctx *ctx, ah_seq *seq);
/* Polls a grid-barrier wait of this sequence makes before it gives up (0: the default, 2^21, about
 * 0.1 s).  A wait that gives up records AH_ERR_SEQ_TIMEOUT at its stage and every later wait of
 * that launch is skipped, so every workgroup still runs to the end and signals each of its
 * stages: the barrier counters stay consistent and the next run is a whole run again.  No
 * counterpart in the reference; for tests of that path. */
int32_t ah_seq_set_spin_limit(ah_seq *seq, uint32_t polls);
/* The sequence's resident grid (workgroups of 512 threads) and its per-workgroup activation LDS. */
int32_t ah_seq_info(const ah_seq *seq, uint32_t *grid, uint32_t *act_bytes);

/* ---- prefill GEMM, N = n_tok > 1 (kern/matmat.rs:134 matmat_q8act) ---- */

/* y[n_tok][n_out] (token-major) = X W^T for X[n_tok][n_in] f32; quantization is a separate
 * in-stream pass into context scratch (grown on demand, never shrunk), which also holds split-K
 * partials.  GEMM calls on one context share that scratch: calls on different streams of the same
 * context must not overlap (use one context per stream for concurrent prefills). */
int32_t ah_gemm_f32_dev(ah_ctx *ctx, const ah_tensor *w, const float *d_x, size_t n_tok,
                        float *d_y, void *stream);
/* ah_gemm_f32_dev that allocates nothing.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The call calls no hipMalloc/hipFree or other allocating
 * routine; its operand and split-K scratch is a 64 MiB static device array the library holds on
 * each GPU until the process ends (ah_gemm_noalloc_scratch_bytes reports the size), and a call
 * that needs more refuses with AH_ERR_SCRATCH_LIMIT before it enqueues anything (at K = 8960,
 * N = 512 it needs about 40 MiB).  Every call on one GPU shares that array and each call writes
 * every scratch byte it reads, so nothing carries over between calls; calls that overlap on one
 * GPU (other streams, other contexts, other threads) race on it and must be serialised by the
 * caller.  Results equal ah_gemm_f32_dev's bit for bit. */
int32_t ah_gemm_f32_noalloc_dev(ah_ctx *ctx, const ah_tensor *w, const float *d_x, size_t n_tok,
                                float *d_y, void *stream);
int32_t ah_gemm_noalloc_scratch_bytes(size_t *bytes);
/* Bytes of device scratch the context holds (grown on demand by the allocating GEMM forms; 0 until
 * one of them runs): lets a caller check that a sequence of calls allocated nothing. */
int32_t ah_ctx_scratch_bytes(const ah_ctx *ctx, size_t *bytes);
/* Same from pre-quantized codes[n_tok][n_in] + scales[n_tok][ceil(n_in/32)]. */
int32_t ah_gemm_q8_dev(ah_ctx *ctx, const ah_tensor *w, const int8_t *d_codes,
                       const int64_t *d_scales, size_t n_tok, float *d_y, void *stream);

/* Design of a type's prefill GEMM.  The reference has one CPU kernel per type (gemm_q8_0,
 * kern/gemm.rs:488-580); here several MFMA designs meet the same contract, selectable per context
 * and type for comparison (results agree within the tolerance, not bit for bit):
 *   AH_GEMM_DESIGN_INT8: v_mfma_i32_32x32x32_i8 exact block dots of the int8 codes, folded with
 *     d * 2^(e_b - E) formed exactly by a bf16 outer-product MFMA (no exponent band); for Q4_K
 *     the dots are per 32-element sub-block on the raw nibbles, folded with d sc_j and, for the
 *     min term, dmin m_j times the token's scaled code sum (two more bf16 outer products);
 *   AH_GEMM_DESIGN_F16: v_mfma_f32_32x32x16_f16 on exact f16 operands (the K-quants' design);
 *   AH_GEMM_DESIGN_AUTO (the default): the F16 design, measured 17-25% faster on MI355X at the
 *     configs[3] shapes (N = 512).
 *   AH_GEMM_DESIGN_F16_TILE: the dequantize-once design for Q4_K, Q2_K and Q3_K: each 256-thread
 *     workgroup owns a 128-row x 128-token tile, converts each weight super-block to exact f16
 *     (sc * q, folded with d and the min term per super-block) once into LDS, and every wave
 *     feeds v_mfma_f32_32x32x16_f16 from that LDS copy and from activation fragments in
 *     registers.
 * Per type: Q8_0 takes AUTO, F16 or INT8; Q4_K takes AUTO (= F16), F16, INT8 or F16_TILE; Q2_K and
 * Q3_K take AUTO (= F16_TILE) or F16, which for these two types serves the prefill as one
 * streaming GEMV per token (the reference's matmat_q8act loop, chart/mod.rs:1955-1975); Q5_0,
 * Q6_K and Q8_K take AUTO or F16.  Any other pairing returns AH_ERR_UNSUPPORTED_QUANT. */
#define AH_GEMM_DESIGN_AUTO 0u
#define AH_GEMM_DESIGN_F16 1u
#define AH_GEMM_DESIGN_INT8 2u
#define AH_GEMM_DESIGN_F16_TILE 3u
int32_t ah_set_gemm_design(ah_ctx *ctx, uint32_t ggml_type, uint32_t design);

/* Grouped prefill: n_parts projections of ONE input (q/k/v, gate/up).  gemm_q8_0_group
 * (kern/gemm.rs:799-818) shares one activation pack over its parts; here one operand pass
 * serves every part, then one GEMM launch per run of same-type parts and one split-K
 * reduction for the parts that split, in order on the stream.  All parts share n_in
 * (AH_ERR_INVALID_ARG otherwise); ggml types and n_out may differ.  d_y[i] is part i's
 * [n_tok][n_out_i] output; each equals what the single-projection call produces for that part. */
int32_t ah_gemm_group_f32_dev(ah_ctx *ctx, size_t n_parts, const ah_tensor *const *w,
                              const float *d_x, size_t n_tok, float *const *d_y, void *stream);
int32_t ah_gemm_group_q8_dev(ah_ctx *ctx, size_t n_parts, const ah_tensor *const *w,
                             const int8_t *d_codes, const int64_t *d_scales, size_t n_tok,
                             float *const *d_y, void *stream);

/* ---- debug: exact integer group dots (the bit-exact quantity of the contract) ---- */

/* ah_gemv_q8_dev that ALSO stores, from inside the same production kernel, the exact integer
 * group dots it folds: d_dots is [n_out][ngroups] int32 with ngroups = ceil(n_in/32) for Q8_0
 * (sum q*xq) and Q4_K (sum nibble*xq), ceil(n_in/16) for Q6_K (sum (u-32)*xq).  These are
 * RowAcc::emit's `dot` (chart/mod.rs:501-514), compared bit for bit with the CPU contract. */
int32_t ah_gemv_q8_dots_dev(ah_ctx *ctx, const ah_tensor *w, const int8_t *d_codes,
                            const int64_t *d_scales, float *d_y, int32_t *d_dots, void *stream);

/* ---- diagnostics ---- */

/* Measures the matrix-core ceiling that bounds the prefill GEMM: a kernel issuing nothing but
 * back-to-back MFMAs (kind 0: v_mfma_i32_32x32x32_i8, kind 1: v_mfma_f32_32x32x16_f16, the
 * instruction the GEMM uses) on every CU, timed with HIP events on the context's stream.
 * Returns tera-ops per second in *tera_ops.  Plays the part of the reference's DP4A ceiling
 * probe (gpu/simt/dp4a.rs:1421-1443), which measures the int8 dot rate of its own device. */
int32_t ah_probe_mfma_peak(ah_ctx *ctx, uint32_t kind, double *tera_ops);

/* ---- status ---- */

/* Synchronize `stream` and return (then clear) the first data-dependent refusal recorded by
 * kernels since the last call, else AH_OK (or AH_ERR_HIP if the stream faulted).  In the
 * reference's order: input conversion (AH_ERR_NONFINITE_INPUT, AH_ERR_INPUT_RANGE, earliest
 * element), then quantization (AH_ERR_FIXED_OVERFLOW: quant_act's None, or a pre-quantized
 * QuantAct that fails dequantizes, chart/mod.rs:128-134), then the outputs (earliest token, then
 * row): AH_ERR_ACCUMULATOR_OVERFLOW where |y| >= 2^63 (the exact sum y * 2^64 leaves i128,
 * ops/matvec.rs:35-37) and AH_ERR_OUTPUT_OVERFLOW where |y| >= 2^31 (round_shift_32 leaves i64,
 * ops/matvec.rs:113-115).  Outputs are classified from the f32 result, so a value within the
 * f32 fold's tolerance of either bound may be classed either way; and an i128 partial sum that
 * overflows and cancels back into range (a refusal of the reference's sequential checked sum)
 * is not seen. */
int32_t ah_sync_status(ah_ctx *ctx, void *stream);

/* ---- host convenience forms (synchronous; copy in and out) ---- */

/* matvec_q8act (chart/mod.rs:1887): codes[n_in], scales[ceil(n_in/32)] host -> y[n_out] host. */
int32_t ah_matvec_q8act(ah_ctx *ctx, const ah_tensor *w, const int8_t *codes,
                        const int64_t *scales, size_t n_codes, float *y);
/* matmat_q8act (kern/matmat.rs:134): codes[n_tok][n_in], scales[n_tok][nb] -> y[n_tok][n_out]. */
int32_t ah_matmat_q8act(ah_ctx *ctx, const ah_tensor *w, const int8_t *codes,
                        const int64_t *scales, size_t n_tok, float *y);
/* quant_act (chart/mod.rs:258) on host Q32.32 input. */
int32_t ah_quant_act(ah_ctx *ctx, const int64_t *x, size_t n, int8_t *codes, int64_t *scales);

#ifdef __cplusplus
}
#endif
#endif
