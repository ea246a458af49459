/*
 * oracle.h -- CPU restatement of the reference's causal GQA prefill attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the Node addon, the
 * JavaScript engine) may include, link or call this code.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py use it, and only as the checker.
 *
 * Reference (read-only, cited as path:line relative to the reference checkout):
 *   src/webgpu/ops.ts:168-241        tiled flash attention shader (the hot path)
 *   src/webgpu/ops.ts:186-193        update_stats (online softmax in mixed f32/f16)
 *   src/webgpu/ops.ts:205-209,219-220 causal + 176-prefix/432-window mask and tile skip
 *   src/webgpu/ops.ts:104-150        QK RMSNorm + RoPE producer (defines the input distribution)
 *   src/webgpu/model.ts:76-83        RoPE table (theta 1e6, f64 -> f32)
 *   src/math/f16.ts:4-25             floatToHalf (reference host encoder, ties away from zero)
 *   src/gguf/quantization.ts:2-9     halfToFloat
 *
 * Pinning status of each function is listed beside its declaration.
 */
#ifndef QATTN_ORACLE_H
#define QATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 codec --------------------------------------------------------------------------- */
/* IEEE binary16 round-to-nearest-even from f32.  Pinned: exhaustive round trip of all 65,536
 * halves, midpoint ties, overflow/subnormal boundaries, cross-check against numpy.float16. */
uint16_t orc_f32_to_f16(float f);
/* binary16 -> f32 (exact).  Pinned: reference KATs tests/quantization.test.ts:5-9 + numpy. */
float orc_f16_to_f32(uint16_t h);
/* The reference's host encoder src/math/f16.ts:4-25: rounds mantissa ties up in magnitude and
 * maps NaN to Inf.  Pinned: equals RNE except on exact ties; KATs for ties, NaN, overflow. */
uint16_t orc_ref_float_to_half(float f);
/* The reference's decoder src/gguf/quantization.ts:2-9 (as f64). */
double orc_ref_half_to_float(uint16_t h);

/* ---- deterministic input generator (restates ops.ts:104-150 + model.ts:76-83) ------------- */
/* i-th output (0-based) of SplitMix64 started at state `seed`.  Pinned: published SplitMix64
 * reference outputs for seed 1234567. */
uint64_t orc_rand_u64(uint64_t seed, uint64_t i);
/* N(0,1) draw for element e (Box-Muller over the pair e>>1, cos for even e, sin for odd e). */
double orc_normal(uint64_t seed, uint64_t e);
/* Seed of one tensor: 0x51574E33_00000000 | config<<16 | layer<<8 | tensor (0 Q, 1 K, 2 V, 3 lengths). */
uint64_t orc_seed(uint32_t config, uint32_t layer, uint32_t tensor);
/* Fill n fp16 N(0,1) values: out[i] = f16((float)normal(seed, i)). */
void orc_gen_normal_f16(uint64_t seed, int64_t n, uint16_t* out);
/* RoPE table [npos][64] cos and sin as f32 computed in f64 (model.ts:76-81). */
void orc_rope_table(int32_t npos, double theta, float* cos_out, float* sin_out);
/* In-place per-head RMSNorm (eps, unit gain when weight==NULL) + NeoX rotate-half RoPE at
 * per-sequence positions (ops.ts:129-147; positions restart at every cu_seqlens boundary).
 * x: fp16 rows of `stride` elements, `heads` vectors of 128 at element offset `col0` of a row. */
void orc_qk_norm_rope(uint16_t* x, int64_t stride, int64_t col0, int32_t heads,
                      const int32_t* cu_seqlens, int32_t nseq, const float* weight,
                      double eps, double theta);
/* Lengths for config 1: 10 + (rand(seed3, i) >> 33) % 141. */
void orc_gen_lengths(uint64_t seed, int32_t n, int32_t lo, int32_t hi, int32_t* out);

/* ---- mask (ops.ts:205-209, 219-220) ------------------------------------------------------- */
enum { ORC_MASK_CAUSAL = 0, ORC_MASK_PREFIX_LOCAL = 1 };
/* Literal reference predicate: q<S && k<=q && k<S && (causal || k<min(S,P) || k+min(S,W)>q).
 * Pinned: closed-form pair counts, brute-force enumeration, torch boolean mask cross-check. */
int orc_retained(int64_t q, int64_t k, int64_t S, int32_t kind, int64_t P, int64_t W);
/* Row-major bitmask of one sequence: word q*ceil(L/32) + k/32, bit k%32. */
void orc_mask_bits(int32_t L, int32_t kind, int32_t P, int32_t W, uint32_t* bits);
/* Number of retained pairs of one sequence, by enumeration. */
int64_t orc_mask_pairs(int32_t L, int32_t kind, int32_t P, int32_t W);
/* Would the reference's 16x16 tiled kernel skip key tile `key_base` for query tile starting at
 * `q_tile_start`?  ops.ts:205-209 literally. */
int orc_ref_tile_skipped(int64_t S, int64_t q_tile_start, int64_t key_base);

/* ---- attention ---------------------------------------------------------------------------- */
/* Shared argument block.  Element strides (halves per token row); V read at v + v_offset. */
typedef struct orc_attn_args {
  const uint16_t* q; const uint16_t* k; const uint16_t* v;
  int64_t q_stride, k_stride, v_stride, v_offset;
  const int32_t* cu_seqlens; int32_t nseq;
  int32_t kind, prefix, window;
} orc_attn_args;

/* Exact attention in f64: O = softmax(mask(Q K^T) / sqrt(128)) V for the listed token rows
 * (rows==NULL: all T rows).  out: [nrows][16][128] doubles.  Pinned: closed forms (V const,
 * Q = 0, single key), torch SDPA float64 with boolean mask, invariants. */
void orc_attention_exact(const orc_attn_args* a, const int64_t* rows, int64_t nrows, double* out);

/* f16-faithful restatement of the reference's tiled kernel ops.ts:194-240: 16-query x 16-key
 * tiles in the same loop order and skip rule, f16 dot4 partials summed in f32, f32 scores and
 * running max, f16 weights / alpha / beta / denominator / accumulator, f16 divide.  WGSL's exp
 * and f16 dot rounding are implementation-defined: this uses correctly rounded f32 exp (via
 * f64) and strict per-operation f16 rounding.  out: fp16 [T][16][128] (row stride o_stride).
 * Pinned: agrees with the f64 oracle to f16 accumulation error; closed forms that are exact in
 * f16 (V constant in {0.5,1,2}, single key) hold bit-exactly. */
void orc_attention_tiled16(const orc_attn_args* a, uint16_t* out, int64_t o_stride);

/* The same restatement for the 16-query tiles tile_begin, tile_begin+tile_step, ... < tile_end of
 * one sequence (all 16 heads): a bounded sample of a long sequence for CPU timing. */
void orc_attention_tiled16_tiles(const orc_attn_args* a, int32_t seq, int64_t tile_begin,
                                 int64_t tile_end, int64_t tile_step, uint16_t* out,
                                 int64_t o_stride);

/* Threads used by the OpenMP loops (0 = runtime default). */
void orc_set_threads(int32_t n);
int32_t orc_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
