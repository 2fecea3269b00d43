/*
 * fence_oracle.h -- scalar CPU restatement of Fence's fused per-layer ops.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP kernels
 * in the product library (libfence_ops.so).  Only the tests, the smoke check
 * and the CPU-baseline leg of bench.py may load it; the product path never
 * calls it and never falls back to it.
 *
 * Each function cites the reference launcher/kernel it restates
 * (paths are relative to the reference repository root).
 *
 * Numerics (deliberate, documented choices):
 *   - fp32 element arithmetic, compiled with -ffp-contract=off and without
 *     fast-math, so every product and sum is rounded exactly once as written;
 *   - row reductions (sum of squares, sum of exponentials) accumulate in
 *     double: the reference's fp32 shared-memory tree order is not
 *     reproducible and double is closer to the exact value;
 *   - transcendentals are glibc powf / sinf / cosf / expf (the reference is
 *     built with --use_fast_math, whose approximate intrinsics cannot be run
 *     here; the parity target is the formula, not that binary);
 *   - fp16 is decoded by an explicit bit routine (signalling NaNs are quieted,
 *     as IEEE-754 conversion and the x86 F16C / AMD v_cvt_f32_f16
 *     instructions do).
 *
 * Parity pinning for every function is listed in the tests
 * (tests/oracle_checks.py); the mutation tests plant mistakes in a copy of
 * this oracle and require that those checks catch each one.
 */
#ifndef FENCE_ORACLE_H
#define FENCE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Q8_0 block: fp16 scale followed by 32 int8 values, 34 bytes, packed.
 * Follows src/kernels/q8_0_types.h:8-17. */
#define FO_QK8_0 32
#define FO_Q8_0_BLOCK_BYTES 34

enum { FO_ROPE_NEOX = 0, FO_ROPE_INTERLEAVED = 1 };

float fo_fp16_to_f32(uint16_t h);

/* a1: src/kernels/ops.cuh:17-51 */
void fo_rms_norm(float* out, const float* x, const float* w, int n, float eps);
/* a2: src/kernels/ops.cuh:54-60 (out aliases x) */
void fo_rms_norm_inplace(float* x, const float* w, int n, float eps);
/* a1 applied to `rows` consecutive rows of length n (prefill composition) */
void fo_rms_norm_rows(float* out, const float* x, const float* w,
                      int64_t rows, int n, float eps);
/* a3: src/kernels/ops.cuh:66-103 */
void fo_rms_norm_per_head(float* x, const float* w, int n_heads, int head_dim,
                          float eps);

/* inverse frequency of pair p: src/kernels/ops.cuh:133 */
void fo_rope_inv_freq(float* inv_freq, int head_dim, float freq_base);
/* rotate one head in place at one position.
 * NeoX pairs (p, p+hd/2): src/kernels/ops.cuh:133-144;
 * interleaved pairs (2p, 2p+1): comment src/kernels/ops.cuh:109-113. */
void fo_rope_head(float* x, int head_dim, int pos, float freq_base, int style);
/* a4: src/kernels/ops.cuh:115-177 (NeoX, Q and K in one call) */
void fo_apply_rope(float* q, float* k, int head_dim, int n_q_heads,
                   int n_kv_heads, int pos, float freq_base);
/* a4/a5 over tokens: q [tokens][n_q_heads][hd], k [tokens][n_kv_heads][hd];
 * position of token t = positions ? positions[t] : pos0 + t. */
void fo_rope_rows(float* q, float* k, int64_t tokens, int n_q_heads,
                  int n_kv_heads, int head_dim, const int32_t* positions,
                  int pos0, float freq_base, int style);

/* a6: src/kernels/ops.cuh:183-202 (out may alias gate) */
void fo_silu_elementwise_mul(float* out, const float* gate, const float* up,
                             int64_t n);

/* a9: src/kernels/ops.cuh:207-251, in place */
void fo_softmax(float* x, int n);
/* a9 on `rows` rows of length n, row stride ld (decode score rows,
 * src/kernels/ops.cuh:357-391 with seq_len = n, stride max_ctx) */
void fo_softmax_rows(float* x, int64_t rows, int n, int64_t ld);
/* causal softmax over [heads][sq][sk]: query i sees keys 0..i+(sk-sq);
 * masked keys are written as exactly 0 (== expf(-inf - m)). */
void fo_softmax_causal(float* x, int64_t heads, int sq, int sk);

/* a10: src/kernels/gemv_q8_0.cuh:12-36 */
void fo_embed_q8_0(float* out, const uint8_t* table, int token_id, int dim);
/* a12: one a10 per token; an id outside [0,vocab) yields a row of quiet NaN.
 * Returns the number of out-of-range ids. */
int64_t fo_embed_q8_0_gather(float* out, const uint8_t* table, int64_t vocab,
                             const int32_t* ids, int64_t tokens, int dim);
/* a12 then a1 on each gathered row */
int64_t fo_embed_q8_0_gather_rms_norm(float* out, const uint8_t* table,
                                      int64_t vocab, const int32_t* ids,
                                      int64_t tokens, int dim, const float* w,
                                      float eps);

/* Q8_0 GEMV, y[M] = W[M x K] x[K]: src/kernels/gemv_q8_0.cuh:40-104
 * (per row: sum over blocks of d * sum_i qs[i] * x[32b+i]), accumulated in
 * double.  K % 32 == 0. */
void fo_gemv_q8_0(const uint8_t* W, const float* x, float* y, int M, int K);

/* Q6_K super-block: ql[128] low nibbles, qh[64] high crumbs, int8 scales[16],
 * fp16 d; 210 bytes, 256 weights.  src/kernels/q6k_types.h:24-35. */
#define FO_QK_K 256
#define FO_Q6K_BLOCK_BYTES 210

/* The 6-bit quant of element i (0..63), src/kernels/q6k_dot.cuh:35-64. */
int fo_q6k_quant(const uint8_t* blk, int i);
/* dot(block, x[256]) with x as binary16 bit patterns, summed exactly in
 * double: sum_i d * scales[i/16] * (q6[i] - 32) * x[i]
 * (src/kernels/q6k_dot.cuh:28-72; the reference tests' CPU golden,
 * tests/test_q6k_dot.cu:40-83). */
double fo_q6k_dot(const uint8_t* blk, const uint16_t* x16);
/* y[M] = W[M x K] x[K] (+ bias[M] if bias), W rows of K/256 Q6_K blocks, x
 * binary16, y fp32: src/kernels/gemv_q6k.cuh:44-151.  K % 256 == 0. */
void fo_gemv_q6k(const uint8_t* W, const uint16_t* x16, const float* bias, float* y,
                 int M, int K);

/* store_kv, src/kernels/ops.cuh:419-443: k_cache[pos*kv_dim + i] =
 * binary16(k[i]), the same for v (caches are binary16 bit patterns). */
void fo_store_kv(uint16_t* k_cache, uint16_t* v_cache, const float* k, const float* v,
                 int pos, int kv_dim);
/* gqa_attention, src/kernels/ops.cuh:320-413, one query position: for query
 * head h (kv head h / (n_q/n_kv)), s_t = (q_h . k_t) * scale over the
 * seq_len cached positions, p = softmax(s) (the -1e30 initial maximum and
 * e * (1/sum) of the reference), out_h = sum_t p_t v_t.  Caches are
 * [max_ctx][n_kv][head_dim] binary16; scale = 1/sqrt(head_dim) rounded to
 * fp32.  Dots and the output sum accumulate in double. */
void fo_gqa_attention(float* out, const float* q, const uint16_t* k_cache,
                      const uint16_t* v_cache, int head_dim, int n_q_heads,
                      int n_kv_heads, int seq_len, int max_ctx);
/* argmax, src/kernels/ops.cuh:467-505, as the reference's one 256-thread
 * block computes it: thread t keeps the first strict maximum of x[t],
 * x[t+256], .. (initial -1e30f, index 0), then a tree over s = 128 .. 1 in
 * which slot u takes slot u+s only if strictly greater.  A tie across
 * threads goes to the thread with the smallest 8-bit bit-reversal, which is
 * not always the lowest index (maxima at 1 and 256 give 256). */
int fo_argmax(const float* x, int n);

/* IEEE binary32 -> binary16, round to nearest, ties to even; overflow -> inf;
 * NaN -> quiet NaN of the same sign.  The reference's __float2half in
 * f32_to_f16 (src/kernels/ops.cuh:448-462) and float_to_half (:274-289). */
uint16_t fo_f32_to_f16(float f);
void fo_f32_to_f16_array(uint16_t* out, const float* in, int64_t n);
/* residual_add, src/kernels/ops.cuh:256-270: x[i] += residual[i] */
void fo_residual_add(float* x, const float* residual, int64_t n);
/* The layer-boundary epilogue of src/model/qwen3.cu:310-325 (and :272-278
 * without a residual), per row of n: hidden += residual (if residual),
 * normed = rms_norm(hidden, w), out16 = f32_to_f16(normed).  normed and out16
 * may each be NULL. */
void fo_residual_rms_norm_f16(float* hidden, const float* residual, const float* w,
                              float* normed, uint16_t* out16, int64_t rows, int n,
                              float eps);
/* src/model/qwen3.cu:332-336: act = silu(gate) * up; out16 = f32_to_f16(act);
 * out (fp32 act) may be NULL. */
void fo_swiglu_f16(uint16_t* out16, float* out, const float* gate, const float* up,
                   int64_t n);

/* a7: per-head RMSNorm of q (weight wq[hd]) and k (wk[hd]) then RoPE,
 * per token (src/model/qwen3.cu:293-299 composed). */
void fo_qk_norm_rope(float* q, float* k, const float* wq, const float* wk,
                     int64_t tokens, int n_q_heads, int n_kv_heads,
                     int head_dim, float eps, const int32_t* positions,
                     int pos0, float freq_base, int style);
/* a8: out_t = RoPE(rms_norm(x_t, w)) viewed as [n_q_heads][hd]; k gets RoPE
 * only (apply_rope's q+k contract, src/kernels/ops.cuh:169). */
void fo_rms_norm_rope(float* out, const float* x, const float* w, float* k,
                      int64_t tokens, int n_q_heads, int n_kv_heads,
                      int head_dim, float eps, const int32_t* positions,
                      int pos0, float freq_base, int style);

/* CPU-baseline timing (fence_oracle_time.c; bench.py's cpu_baseline leg):
 * `reps` passes of the elementwise stage of BASELINE configs[4] on caller
 * buffers -- fo_softmax_causal over [heads][sq][sk], fo_silu_elementwise_mul
 * over n elements into act, fo_rope_rows over `tokens` tokens at
 * positions[t] -- with the seconds spent in each of the three accumulated
 * into secs[0..2] (CLOCK_MONOTONIC around each call). */
void fo_time_elementwise_stage(double secs[3], int reps, float* scores, int64_t heads, int sq,
                               int sk, float* act, const float* gate, const float* up, int64_t n,
                               float* q, float* k, int64_t tokens, int n_q_heads, int n_kv_heads,
                               int head_dim, const int32_t* positions, float freq_base, int style);

#ifdef __cplusplus
}
#endif

#endif /* FENCE_ORACLE_H */
