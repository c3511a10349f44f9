/*
 * ah_oracle.h -- CPU restatement of apeiron's quantized-projection contract.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker (or, for the
 * CPU baseline, as the thing timed on the host).  The product path never links,
 * loads or calls it.
 *
 * Every function cites the reference file:line (relative to the apeiron tree) whose
 * algorithm it restates.  The status codes mirror include/apeiron_hip.h one for one.
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   aho_f16_to_fixed      exhaustive over all 65536 words vs exact rational decode
 *   aho_to_q32            exact rational rounding on edge + random f32 words
 *   aho_act_scale         reference sample table (kern/pow2.rs:105-135) + brute force
 *   aho_quant_act         reference KATs (chart/tests.rs:373-415) + invariants
 *   aho_dequant_row       reference unpack KATs (format/quant.rs:784-899) + big-int decode
 *   aho_matvec_fixed      reference 2x2 KAT (engine/tests.rs:389-407) + big-int brute force
 *   aho_block_dots        big-int brute force on the same payloads
 *   aho_matvec_q8act_fast bit-equal to aho_matvec_fixed on every tested payload
 *   aho_fixed_exp         reference KATs (fixed_exp.rs zero_and_boundaries), accuracy against
 *                         exp on a dense grid and monotonicity (fixed_exp.rs tests)
 *   aho_silu_fixed        reference KATs (engine/tests.rs:949-963) + the closed form
 *                         v / (1 + e^-v) within the exp tolerance + saturation bounds
 *   aho_swiglu            exact big-int product rounding on random operands
 */
#ifndef AH_ORACLE_H
#define AH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: identical values to include/apeiron_hip.h (AH_*). */
enum {
    AHO_OK = 0,
    AHO_ERR_SHAPE_MISMATCH = 1,      /* MatvecError::ShapeMismatch                 */
    AHO_ERR_ROW_LENGTH = 2,          /* MatvecError::RowLength                     */
    AHO_ERR_SHORT_PAYLOAD = 3,       /* MatvecError::ShortPayload                  */
    AHO_ERR_LENGTH_OVERFLOW = 4,     /* MatvecError::LengthOverflow                */
    AHO_ERR_UNSUPPORTED_QUANT = 5,   /* MatvecError::UnsupportedQuant              */
    AHO_ERR_NONFINITE_SCALE = 6,     /* MatvecError::Dequant(NonFiniteScale)       */
    AHO_ERR_FIXED_OVERFLOW = 7,      /* MatvecError::Dequant(FixedOverflow)        */
    AHO_ERR_ACCUMULATOR_OVERFLOW = 8,/* MatvecError::AccumulatorOverflow           */
    AHO_ERR_OUTPUT_OVERFLOW = 9,     /* MatvecError::OutputOverflow                */
    AHO_ERR_NONFINITE_INPUT = 10,    /* F32Error::NonFinite (f32 boundary)         */
    AHO_ERR_INPUT_RANGE = 11,        /* F32Error::OutOfRange (f32 boundary)        */
    AHO_ERR_FFN_OVERFLOW = 12,       /* FfnError::Overflow                         */
    AHO_ERR_EXP_RANGE = 13,          /* FfnError::ExpOutOfRange (ExpError)         */
    AHO_ERR_ZERO_DENOMINATOR = 14         /* FfnError::ZeroDenominator                  */
};

enum { AHO_Q5_0 = 6, AHO_Q8_0 = 8, AHO_Q2_K = 10, AHO_Q3_K = 11, AHO_Q4_K = 12, AHO_Q6_K = 14 };

/* (weights per block, bytes per block) -- format/quant.rs:129-147.  0 on unknown type. */
int aho_block_geom(uint32_t ggml_type, size_t *qk, size_t *block_bytes);
/* Row stride ceil(n_in/qk)*block_bytes -- ops/matvec.rs:167-168. */
int aho_row_bytes(uint32_t ggml_type, size_t n_in, size_t *row_bytes);

/* num/dequant.rs:25-41 */
int aho_f16_to_fixed(uint16_t h, int64_t *out);
/* num/fp.rs:186-230 + num/f32_convert.rs:44-49 */
int aho_to_q32(uint32_t f32_bits, int64_t *out);
/* kern/pow2.rs:11-39; returns 0 and writes *out, or 1 for None. */
int aho_act_scale(uint64_t absmax, uint64_t *out);
/* chart/mod.rs:235-334 (with QuantAct::dequantizes, :105-134) */
int aho_quant_act(const int64_t *x, size_t n, int8_t *codes, int64_t *scales);
/* a2 then a3: every f32 through to_q32, then quant_act. */
int aho_quant_act_f32(const float *x, size_t n, int8_t *codes, int64_t *scales);
/* QuantAct::dequant (chart/mod.rs:186-209): x_hat = S_b * xq, or FIXED_OVERFLOW. */
int aho_dequant_act(const int8_t *codes, const int64_t *scales, size_t n, int64_t *xhat);

/* num/dequant.rs:99-122 for Q8_0 (:315-351), Q2_K (:395-462), Q3_K (:464-512), Q4_K (:514-617),
 * Q6_K (:619-671).
 * row must hold ceil(n/qk) whole blocks. */
int aho_dequant_row(uint32_t ggml_type, const uint8_t *row, size_t row_len, size_t n,
                    int64_t *out);

/* ops/matvec.rs:149-222 in exact __int128 arithmetic. */
int aho_matvec_fixed(uint32_t ggml_type, const uint8_t *raw, size_t raw_len, size_t n_out,
                     size_t n_in, const int64_t *x, size_t x_len, int64_t *y);

/* chart/mod.rs:1887-1925: matvec_fixed on QuantAct::dequant, the contract every fast kernel
 * equals bit for bit.  n_codes is QuantAct::len. */
int aho_matvec_q8act(uint32_t ggml_type, const uint8_t *raw, size_t raw_len, size_t n_out,
                     size_t n_in, const int8_t *codes, const int64_t *scales, size_t n_codes,
                     int64_t *y);

/* Exact per-group integer dots of one row against quantized activation codes.
 *   Q8_0: dots[b] = sum_{l<32} q*xq over 32-block b                (ceil(K/32) entries)
 *   Q5_0: dots[b] = sum_{l<32} (q-16)*xq over 32-block b           (ceil(K/32) entries)
 *   Q4_K: dots[j] = sum nibble*xq over 32-sub-block j              (ceil(K/32) entries)
 *   Q6_K: dots[g] = sum (u-32)*xq over 16-group g                  (ceil(K/16) entries)
 *   Q2_K: dots[g] = sum q*xq over 16-group g, q in 0..3            (ceil(K/16) entries)
 *   Q3_K: dots[g] = sum c*xq over 16-group g, c in -4..3           (ceil(K/16) entries)
 * xsums[b] = sum xq over 32-block b (ceil(K/32) entries).  Lanes >= K contribute nothing.
 * The factorisation is chart/mod.rs:11-16 (RowAcc::emit :501-514). */
int aho_block_dots(uint32_t ggml_type, const uint8_t *row, size_t row_len, size_t n_in,
                   const int8_t *codes, int32_t *dots, int32_t *xsums);

/* Sum_i |w_i * xhat_i| for each of n_out rows, in real units (Q32.32 products * 2^-64),
 * the normaliser of the parity tolerance. */
int aho_row_absdot(uint32_t ggml_type, const uint8_t *raw, size_t raw_len, size_t n_out,
                   size_t n_in, const int8_t *codes, const int64_t *scales, double *out);

/* The reference's fast CPU path restated for host timing: chart row kernels (block dot +
 * i128 fold, chart/mod.rs:501-514, x86.rs cores) over contiguous row chunks on a thread pool
 * (chart/ffn.rs:667-727); Q8_0, Q5_0 and Q4_K rows two at a time (tiled2, x86.rs:782-1192), the
 * 32-lane dots on AVX-VNNI vpdpbusd where the host has it, else AVX2 vpmaddubsw/vpmaddwd
 * (x86.rs:74-85, 175-205).  Bit-equal to aho_matvec_q8act; falls back to it when the fast bound
 * (chart/mod.rs:336-383) fails. */
int aho_matvec_q8act_fast(uint32_t ggml_type, const uint8_t *raw, size_t raw_len, size_t n_out,
                          size_t n_in, const int8_t *codes, const int64_t *scales, int64_t *y,
                          int n_threads);
/* kern/matmat.rs:134 semantics: column c of y (n_tok x n_out, token-major) equals
 * aho_matvec_q8act on token c.  Routing as matmat_q8act's (matmat.rs:140-180): Q4_K / Q6_K widths
 * that are not whole super-blocks run one aho_matvec_q8act_fast per column (the per-column path,
 * matmat.rs:392-413); otherwise row pairs are tiled over threads, each pair's blocks decoded once
 * and dotted against every column (the k-column form of chart/kcols.rs). */
int aho_matmat_q8act_fast(uint32_t ggml_type, const uint8_t *raw, size_t raw_len, size_t n_out,
                          size_t n_in, size_t n_tok, const int8_t *codes, const int64_t *scales,
                          int64_t *y, int n_threads);

/* The FFN's SwiGLU step (ah_oracle_ffn.c). */
/* numeric/fixed_exp.rs:120-131: exp(x) in Q32.32, x in [-16, 21] * 2^32, else AHO_ERR_EXP_RANGE. */
int aho_fixed_exp(int64_t x, int64_t *out);
/* engine/ops/silu.rs:18-60 */
int aho_silu_fixed(int64_t v, int64_t *out);
/* engine/chart/ffn.rs:246-252: h = round_shift_32(silu_fixed(gate) * up) */
int aho_swiglu(int64_t gate, int64_t up, int64_t *h);
/* to_q32 of f32 gate/up, aho_swiglu, then aho_quant_act: the down projection's QuantAct.
 * h (optional, n entries) receives the hidden Q32.32 values. */
int aho_swiglu_quant_f32(const float *gate, const float *up, size_t n, int8_t *codes,
                         int64_t *scales, int64_t *h);

/* 1 when the host has AVX2 (the fast cores), else 0 (portable loops are used). */
int aho_has_avx2(void);

/* The cores the fast path runs: portable loops, AVX2 dots, or AVX-VNNI dots. */
#define AHO_CPU_PORTABLE 0
#define AHO_CPU_AVX2 1
#define AHO_CPU_VNNI 2
/* The path in use: the host's best unless forced. */
int aho_cpu_path(void);
/* Forces a path (clamped to what the host has; negative: the host's best) and returns the path
 * now in use (tests run every form the host offers). */
int aho_set_cpu_path(int path);

#ifdef __cplusplus
}
#endif
#endif
