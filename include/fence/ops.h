/*
 * fence/ops.h -- C ABI of the MI355X (gfx950) fused per-layer ops.
 *
 * This is the drop-in boundary for the reference's header-only CUDA launchers
 * (src/kernels/ops.cuh, src/kernels/gemv_q8_0.cuh of
 * eeea2222/-Damn-Low-Level-Fence-Inference-version-1).  Every entry point
 * takes caller-owned device pointers and a HIP stream, launches
 * asynchronously on that stream and returns an int status.
 *
 * Conventions (all entry points):
 *   - returns FENCE_SUCCESS (0), FENCE_ERROR_INVALID_VALUE (22 = EINVAL) for a
 *     bad shape, a null pointer or a pointer that is not 4-byte aligned
 *     (checked on the host before anything is launched), or
 *     FENCE_ERROR_HIP_BASE + hipError_t when the launch itself fails;
 *   - never allocates, never synchronises, never exits; no global mutable
 *     state (only per-thread caches), so calls are re-entrant from any host
 *     thread;
 *   - 16-byte aligned rows take the 128-bit vector kernels; other alignments
 *     take scalar kernels with the same results (not an error);
 *   - in-place forms the reference's callers rely on keep working:
 *     rms_norm(out == x) and silu_elementwise_mul(out == gate or out == up).
 *   - fp32 results agree with the reference formulas to 1e-5 of the row's
 *     largest magnitude; Q8_0 dequantisation is bit-exact.
 *
 * Including this header from a non-HIP compiler needs -D__HIP_PLATFORM_AMD__
 * (the usual requirement of hip_runtime_api.h).
 */
#ifndef FENCE_OPS_H
#define FENCE_OPS_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    FENCE_SUCCESS = 0,
    FENCE_ERROR_INVALID_VALUE = 22,
    /* model files and the host forward (fence/gguf.h, fence/model.h) */
    FENCE_ERROR_NOT_FOUND = 2,       /* no such tensor or metadata key */
    FENCE_ERROR_OUT_OF_MEMORY = 12,  /* host or device allocation failed */
    FENCE_ERROR_BAD_FILE = 74,       /* not a readable, well-formed GGUF file */
    FENCE_ERROR_TYPE_MISMATCH = 75,  /* metadata value of another type */
    FENCE_ERROR_UNSUPPORTED = 95,    /* a model this forward does not run */
    FENCE_ERROR_HIP_BASE = 1000
};

/* RoPE pairing.  NEOX pairs (p, p + head_dim/2), as the reference's code
 * (src/kernels/ops.cuh:138-139); INTERLEAVED pairs (2p, 2p+1), as the
 * comment above it (src/kernels/ops.cuh:109-113). */
enum {
    FENCE_ROPE_NEOX = 0,
    FENCE_ROPE_INTERLEAVED = 1
};

/* Q8_0 block: fp16 scale then 32 int8 values, 34 bytes, no padding
 * (src/kernels/q8_0_types.h:8-17). */
#define FENCE_QK8_0 32
#define FENCE_Q8_0_BLOCK_BYTES 34

/* Arrival counters of fence_gqa_attention_qk_f16_arrive: uint32 words per
 * query head (each counter has a 256-byte slot of its own). */
#define FENCE_ARRIVE_WORDS_PER_HEAD 64

/* ---------------------------------------------------------------------------
 * One-to-one replacements of the reference launchers (same argument order and
 * meaning; the stream argument is required in the C ABI).
 * ------------------------------------------------------------------------ */

/* Replaces rms_norm, src/kernels/ops.cuh:47-51.
 * out[i] = w[i] * x[i] * rsqrt(mean(x^2) + eps); out may equal x. */
int fence_rms_norm(float* out, const float* x, const float* w, int n,
                   float eps, hipStream_t stream);

/* Replaces rms_norm_inplace, src/kernels/ops.cuh:54-60. */
int fence_rms_norm_inplace(float* x, const float* w, int n, float eps,
                           hipStream_t stream);

/* Replaces rms_norm_per_head, src/kernels/ops.cuh:97-103.
 * x [n_heads][head_dim] normalised per head in place with w[head_dim]. */
int fence_rms_norm_per_head(float* x, const float* w, int n_heads,
                            int head_dim, float eps, hipStream_t stream);

/* Replaces apply_rope, src/kernels/ops.cuh:169-177 (NeoX pairing, one
 * position for all heads).  q [n_q_heads][head_dim], k [n_kv_heads][head_dim]
 * rotated in place; head_dim even and <= 256. */
int fence_apply_rope(float* q, float* k, int head_dim, int n_q_heads,
                     int n_kv_heads, int pos, float freq_base,
                     hipStream_t stream);

/* Replaces silu_elementwise_mul, src/kernels/ops.cuh:197-202.
 * out[i] = gate[i] / (1 + exp(-gate[i])) * up[i]; out may equal gate or up. */
int fence_silu_elementwise_mul(float* out, const float* gate, const float* up,
                               int n, hipStream_t stream);

/* Replaces softmax, src/kernels/ops.cuh:248-251 (in place, one vector). */
int fence_softmax(float* x, int n, hipStream_t stream);

/* Replaces embed_q8_0, src/kernels/gemv_q8_0.cuh:31-36.
 * out[dim] = dequantised row token_id of the Q8_0 table `weight`
 * ([vocab][dim/32] blocks).  dim % 32 == 0.  Like the reference this form
 * has no vocab argument and cannot check token_id < vocab; use
 * fence_embed_q8_0_gather for checked lookups. */
int fence_embed_q8_0(float* out, const void* weight, int token_id, int dim,
                     hipStream_t stream);

/* Replaces gemv_q8_0, src/kernels/gemv_q8_0.cuh:99-104 (the tied LM head,
 * src/model/qwen3.cu:261).  y[M] = W x for a Q8_0 matrix W of M rows of K/32
 * blocks and fp32 x[K]:  y[r] = sum_b d_b * sum_i qs_b[i] * x[32b + i].
 * K % 32 == 0 and W 2-byte aligned (block_q8_0 holds an fp16), else
 * FENCE_EINVAL; K == 0 writes zeros.  Summation order differs from the
 * reference's; results agree within fp32 rounding of the dot products. */
int fence_gemv_q8_0(const void* W, const float* x, float* y, int M, int K,
                    hipStream_t stream);

/* Replaces gemv_q6k, src/kernels/gemv_q6k.cuh:89-102 (every projection of a
 * decode step, src/model/qwen3.cu:281-337).  y[M] = W x for a Q6_K matrix W
 * of M rows of K/256 blocks (block_q6_K, 210 bytes) and binary16 x[K]:
 *   y[r] = sum_b d_b * sum_i scales_b[i/16] * (q6_b[i] - 32) * x[256b + i].
 * K % 256 == 0, W and x 2-byte aligned, else FENCE_ERROR_INVALID_VALUE. */
int fence_gemv_q6k(const void* W, const void* x, float* y, int M, int K,
                   hipStream_t stream);

/* Replaces gemv_q6k_bias, src/kernels/gemv_q6k.cuh:140-151:
 * y[r] = (W x)[r] + bias[r] (fp32 add), for the q/k/v biases of
 * src/model/qwen3.cu:280-287. */
int fence_gemv_q6k_bias(const void* W, const void* x, const float* bias, float* y,
                        int M, int K, hipStream_t stream);

/* Replaces gqa_attention, src/kernels/ops.cuh:320-413 (src/model/qwen3.cu:
 * 304-305): attention of one query position over the seq_len cached
 * positions.  q [n_q_heads][head_dim] fp32; caches [max_ctx][n_kv_heads]
 * [head_dim] binary16; attn_out [n_q_heads][head_dim] fp32.  score_buf holds
 * n_q_heads * max_ctx floats, as in the reference; it is used as scratch
 * (split-sequence partials) and its contents afterwards are unspecified.
 * scale = 1/sqrt(head_dim) in fp32.  seq_len 0 writes zeros; seq_len >
 * max_ctx or n_q_heads % n_kv_heads != 0 is FENCE_ERROR_INVALID_VALUE.  Calls
 * that share a score_buf must not overlap. */
int fence_gqa_attention(float* attn_out, const float* q, const void* k_cache,
                        const void* v_cache, int head_dim, int n_q_heads,
                        int n_kv_heads, int seq_len, int max_ctx, float* score_buf,
                        hipStream_t stream);

/* Replaces store_kv, src/kernels/ops.cuh:435-443 (src/model/qwen3.cu:303):
 * k_cache[pos][i] = binary16(k[i]), v_cache[pos][i] = binary16(v[i]), i <
 * kv_dim.  pos outside [0, max_ctx) is FENCE_ERROR_INVALID_VALUE. */
int fence_store_kv(void* k_cache, void* v_cache, const float* k, const float* v,
                   int pos, int kv_dim, int max_ctx, hipStream_t stream);

/* Replaces argmax, src/kernels/ops.cuh:467-505 (greedy sampling):
 * *result = the index the reference's 256-thread block returns: the largest
 * of x[0..n) above -1e30 (NaN never wins); on a tie, the thread t = i mod 256
 * with the smallest 8-bit bit-reversal, then the lowest index (maxima at 1 and
 * 256 give 256, at 1 and 2 give 2); 0 if nothing is above -1e30 or n == 0.
 * One workgroup, no scratch memory. */
int fence_argmax(const float* x, int* result, int n, hipStream_t stream);

/* fence_argmax over many workgroups (same result): the first kernel writes
 * one 8-byte partial per workgroup into `workspace` (8-byte aligned; up to
 * 1024 partials, fewer if workspace_bytes is smaller, at least one), a second
 * one-workgroup kernel reduces them.  The reference's argmax signature has no
 * scratch argument; a caller that owns a buffer (the model's decode
 * scratch) uses this form.  EINVAL if workspace is null or under 8 bytes. */
int fence_argmax_ws(const float* x, int* result, int n, void* workspace, int64_t workspace_bytes,
                    hipStream_t stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): fence_argmax_ws with its partials in the library's own
 * static device scratch (8 KiB, up to 1024 partials; every n fits) instead of
 * a workspace.  Allocates nothing.  Each GPU holds one scratch for the life of
 * the process and every call on that GPU shares it: calls that overlap on one
 * GPU (two streams or threads at once) race; calls ordered on one stream do
 * not.  The stream must belong to the current device (EINVAL otherwise): the
 * scratch address used is the current device's.  Same index as fence_argmax. */
int fence_argmax_noalloc(const float* x, int* result, int n, hipStream_t stream);

/* Replaces residual_add, src/kernels/ops.cuh:265-270: x[i] += residual[i]. */
int fence_residual_add(float* x, const float* residual, int n, hipStream_t stream);

/* Replaces f32_to_f16, src/kernels/ops.cuh:457-462, and float_to_half,
 * :284-289 (the same operation): out[i] = binary16(in[i]), round to nearest
 * even, overflow to inf, NaN to a quiet NaN.  out holds n binary16 values
 * (__half / _Float16), 2-byte aligned. */
int fence_f32_to_f16(void* out, const float* in, int n, hipStream_t stream);

/* Replaces half_to_float, src/kernels/ops.cuh:303-308: out[i] = in[i] (exact). */
int fence_f16_to_f32(float* out, const void* in, int n, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Batched and fused forms.  These compose the reference's single-row ops over
 * many tokens (its prefill is a per-token loop, src/model/qwen3.cu:478-481)
 * and fuse neighbouring ops so intermediates stay in registers.
 *
 * Token positions: positions[t] if `positions` (device, int32[tokens]) is not
 * NULL, else pos0 + t.
 * ------------------------------------------------------------------------ */

/* rms_norm on each of `rows` rows of length n (src/kernels/ops.cuh:17-51
 * per row).  out may equal x. */
int fence_rms_norm_rows(float* out, const float* x, const float* w,
                        int64_t rows, int n, float eps, hipStream_t stream);

/* RoPE over tokens: q [tokens][n_q_heads][head_dim],
 * k [tokens][n_kv_heads][head_dim] (k may be NULL when n_kv_heads == 0),
 * style FENCE_ROPE_NEOX or FENCE_ROPE_INTERLEAVED (apply_rope,
 * src/kernels/ops.cuh:115-177, per token). */
int fence_rope(float* q, float* k, int64_t tokens, int n_q_heads,
               int n_kv_heads, int head_dim, const int32_t* positions,
               int pos0, float freq_base, int style, hipStream_t stream);

/* Per-head RMSNorm of q (weight q_norm_w[head_dim]) and k (k_norm_w) fused
 * with RoPE, per token: the sequence rms_norm_per_head(q), rms_norm_per_head(k),
 * apply_rope of src/model/qwen3.cu:293-299 in one pass over q and k. */
int fence_qk_norm_rope(float* q, float* k, const float* q_norm_w,
                       const float* k_norm_w, int64_t tokens, int n_q_heads,
                       int n_kv_heads, int head_dim, float eps,
                       const int32_t* positions, int pos0, float freq_base,
                       int style, hipStream_t stream);

/* fence_gqa_attention with its conversion for the o projection
 * (src/model/qwen3.cu:305-310: gqa_attention, then f32_to_f16 of attn_out)
 * in the same launches: out_f16 [n_q_heads][head_dim] = binary16 of the
 * result; attn_out (fp32) may be NULL.  score_buf_floats is score_buf's size
 * in floats (0: the reference's n_q_heads * max_ctx).  A larger buffer lets
 * the sequence be split over more workgroups (partials of n_q_heads * 130
 * floats per split); with the reference's size the result is bit-identical to
 * fence_gqa_attention + fence_f32_to_f16. */
int fence_gqa_attention_f16(float* attn_out, void* out_f16, const float* q,
                            const void* k_cache, const void* v_cache, int head_dim,
                            int n_q_heads, int n_kv_heads, int seq_len, int max_ctx,
                            float* score_buf, int64_t score_buf_floats,
                            hipStream_t stream);

/* fence_qk_norm_rope, then store_kv of the rotated k and of v, in one pass
 * (src/model/qwen3.cu:292-303): after the norm and RoPE of token t's q and k
 * (both still written in fp32), its k and v [n_kv_heads*head_dim] are
 * written as binary16 into row pos_t of k_cache / v_cache
 * [max_ctx][n_kv_heads*head_dim] (store_kv, src/kernels/ops.cuh:419-443),
 * bit-identical to the separate calls.  v: [tokens][n_kv_heads][head_dim].
 * q_norm_w and k_norm_w both NULL: RoPE only (the reference skips QK-norm
 * when a model has no norm weights, src/model/qwen3.cu:293).  Positions from
 * pos0 must lie in [0, max_ctx); a device position outside it stores
 * nothing. */
int fence_qk_norm_rope_store_kv(float* q, float* k, const float* v,
                                const float* q_norm_w, const float* k_norm_w,
                                void* k_cache, void* v_cache, int max_ctx,
                                int64_t tokens, int n_q_heads, int n_kv_heads,
                                int head_dim, float eps, const int32_t* positions,
                                int pos0, float freq_base, int style,
                                hipStream_t stream);

/* One decode token's attention block from its unprepared q, k and v
 * (src/model/qwen3.cu:292-310): fence_qk_norm_rope_store_kv for the token at
 * position pos (one token), then fence_gqa_attention_f16 over seq_len =
 * pos + 1 -- the same outputs and cache rows, bit for bit.  With head_dim
 * 128 and 16-byte aligned operands it is one attention launch (plus the merge
 * of its splits): every workgroup applies QK-norm and RoPE to its own q heads,
 * and the ones that attend to position pos prepare its k and v themselves
 * and write the cache row; otherwise it makes the two calls.  q and k are
 * inputs that may be overwritten (the two calls leave the prepared values
 * there; the one launch leaves them as they were).  style:
 * FENCE_ROPE_NEOX or FENCE_ROPE_INTERLEAVED. */
int fence_gqa_attention_qk_f16(float* attn_out, void* out_f16, float* q, float* k,
                               const float* v, const float* q_norm_w,
                               const float* k_norm_w, void* k_cache, void* v_cache,
                               int head_dim, int n_q_heads, int n_kv_heads, int pos,
                               int max_ctx, float eps, float freq_base, int style,
                               float* score_buf, int64_t score_buf_floats,
                               hipStream_t stream);

/* fence_gqa_attention_qk_f16 in one launch where it would take two: no
 * counterpart in the reference (it replaces the same qwen3.cu:292-310 chain).
 * The last workgroup to finish the positions of a group of query heads merges
 * that group's split partials itself, instead of a second kernel merging all
 * of them.  arrive: n_q_heads * FENCE_ARRIVE_WORDS_PER_HEAD uint32 words that
 * the caller zeroes once before the first call; every call leaves them zero.  Outputs and cache rows
 * are bit-identical to fence_gqa_attention_qk_f16's.  Calls that overlap
 * (other streams) must not share arrive or score_buf. */
int fence_gqa_attention_qk_f16_arrive(float* attn_out, void* out_f16, float* q, float* k,
                                      const float* v, const float* q_norm_w,
                                      const float* k_norm_w, void* k_cache, void* v_cache,
                                      int head_dim, int n_q_heads, int n_kv_heads, int pos,
                                      int max_ctx, float eps, float freq_base, int style,
                                      float* score_buf, int64_t score_buf_floats,
                                      uint32_t* arrive, hipStream_t stream);

/* out_t = RoPE(rms_norm(x_t, w)) for x [tokens][n_q_heads*head_dim],
 * w [n_q_heads*head_dim], the normalised row viewed as n_q_heads heads; k
 * (may be NULL) gets RoPE only.  out may equal x. */
int fence_rms_norm_rope(float* out, const float* x, const float* w, float* k,
                        int64_t tokens, int n_q_heads, int n_kv_heads,
                        int head_dim, float eps, const int32_t* positions,
                        int pos0, float freq_base, int style,
                        hipStream_t stream);

/* silu_elementwise_mul with a 64-bit element count. */
int fence_swiglu(float* out, const float* gate, const float* up, int64_t n,
                 hipStream_t stream);

/* softmax on `rows` rows of n values, row stride ld >= n (the decode
 * attention softmax over seq_len scores per head, src/kernels/ops.cuh:357-391,
 * scores stride max_ctx).  In place. */
int fence_softmax_rows(float* x, int64_t rows, int n, int64_t ld,
                       hipStream_t stream);

/* Causal softmax over x [heads][sq][sk] in place: query i sees keys
 * 0 .. i + (sk - sq); the masked keys are not read and are written as 0. */
int fence_softmax_causal(float* x, int64_t heads, int sq, int sk,
                         hipStream_t stream);

/* Q8_0 embedding gather: out [tokens][dim] = rows ids[t] (device int32) of
 * the table [vocab][dim/32] blocks.  An id outside [0, vocab) is not read and
 * yields a row of quiet NaN.  Bit-exact with embed_q8_0 per id. */
int fence_embed_q8_0_gather(float* out, const void* table, int64_t vocab,
                            const int32_t* ids, int64_t tokens, int dim,
                            hipStream_t stream);

/* Q8_0 gather fused with rms_norm (weight w[dim]) on each gathered row. */
int fence_embed_q8_0_gather_rms_norm(float* out, const void* table,
                                     int64_t vocab, const int32_t* ids,
                                     int64_t tokens, int dim, const float* w,
                                     float eps, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Host-side helpers (no device work).
 * ------------------------------------------------------------------------ */

/* The layer-boundary epilogue (src/model/qwen3.cu:310-325: residual_add,
 * rms_norm, f32_to_f16) in one pass, on `rows` rows of n:
 * hidden += residual (skipped if residual is NULL; the sum stays in hidden and
 * is the next sub-block's residual);  normed = rms_norm(hidden,
 * w, eps);  out_f16 = binary16(normed) (round to nearest even).  normed or
 * out_f16 may be NULL, not both; normed must not be hidden when residual is
 * given.  Without a residual it is qwen3.cu:274-278 (rms_norm, f32_to_f16). */
int fence_residual_rms_norm_f16(float* hidden, const float* residual, const float* w,
                                float* normed, void* out_f16, int64_t rows, int n,
                                float eps, hipStream_t stream);

/* SwiGLU with its conversion for the down projection (src/model/qwen3.cu:
 * 332-336): act = silu(gate) * up; out_f16 = binary16(act); out (fp32 act) may
 * be NULL. */
int fence_swiglu_f16(void* out_f16, float* out, const float* gate, const float* up,
                     int64_t n, hipStream_t stream);

/* Several Q6_K GEMVs that share x and K in one launch: y[i] = W[i] x
 * (+ bias[i]) for i < n <= 4 -- the q, k and v projections of
 * src/model/qwen3.cu:281-289 as one launch.  W, y and M are host arrays of n
 * entries; bias is NULL or a host array whose entries may be NULL.  Each y[i]
 * is bit-identical to fence_gemv_q6k(_bias) on the same operands. */
int fence_gemv_q6k_multi(int n, const void* const* W, float* const* y,
                         const float* const* bias, const int* M, const void* x,
                         int K, hipStream_t stream);

/* The gate and up projections with SwiGLU and its conversion
 * (src/model/qwen3.cu:328-336) in one launch: act[r] = silu(W_gate[r] . x) *
 * (W_up[r] . x); out_f16 = binary16(act); out (fp32 act) may be NULL.
 * Bit-identical to fence_gemv_q6k on each matrix, then fence_swiglu_f16. */
int fence_gemv_q6k_swiglu_f16(const void* W_gate, const void* W_up, const void* x,
                              void* out_f16, float* out, int M, int K,
                              hipStream_t stream);

/* The input row of a projection as the layer boundary makes it
 * (src/model/qwen3.cu:267-278 and 310-325): h = hidden + residual (hidden
 * alone when residual is NULL), x = binary16(rms_norm(h, weight, eps)). */
typedef struct {
    const float* hidden;   /* [K] */
    const float* residual; /* [K] or NULL */
    float* hidden_out;     /* [K]: receives h; required with residual, unused without */
    const float* weight;   /* [K] */
    void* x_f16;           /* [K] binary16: receives x */
    float eps;
} fence_rms_input;

/* fence_gemv_q6k_multi with x computed from `in`: the same results, bit for
 * bit, as fence_residual_rms_norm_f16 on a copy of hidden (into hidden_out and
 * x_f16) followed by fence_gemv_q6k_multi on x_f16 -- and one launch where
 * the norm's vector kernel would run and K <= 8192: every workgroup of the
 * GEMV normalises the row in its prologue.  hidden_out and x_f16 must not
 * overlap hidden, residual or weight (so h cannot be formed in place), nor
 * each other.  K > 0. */
int fence_gemv_q6k_multi_rms(int n, const void* const* W, float* const* y,
                             const float* const* bias, const int* M,
                             const fence_rms_input* in, int K, hipStream_t stream);

/* fence_gemv_q6k_swiglu_f16 with x computed from `in`, as above (one launch
 * up to K = 4096; beyond, the norm kernel and then the pair). */
int fence_gemv_q6k_swiglu_rms_f16(const void* W_gate, const void* W_up,
                                  const fence_rms_input* in, void* out_f16, float* out,
                                  int M, int K, hipStream_t stream);

/* inv_freq[p] = 1.0f / powf(freq_base, (float)(2p) / (float)head_dim) for
 * p < head_dim/2 (src/kernels/ops.cuh:133), computed on the host: the RoPE
 * kernels receive exactly these values. */
int fence_rope_inv_freq(float* inv_freq, int head_dim, float freq_base);

/* Kernel timing: the next kernel this host thread launches through this
 * library records `start` and `stop` (events from hipEventCreate) at its own
 * dispatch start and end (hipExtLaunchKernel), so hipEventElapsedTime gives
 * the kernel's execution time without queueing or dispatch latency -- the
 * interval a kernel-trace profiler reports.  One-shot; NULL, NULL cancels.
 * No counterpart in the reference (it has no timing facility); used by the
 * benchmark. */
int fence_time_next_launch(hipEvent_t start, hipEvent_t stop);

/* The same over the next `count` launches of this thread (an entry point
 * that launches several kernels): start at the first kernel's start, stop at
 * the last one's end.  count < 1 is FENCE_ERROR_INVALID_VALUE. */
int fence_time_next_launches(hipEvent_t start, hipEvent_t stop, int count);

/* Calibration stream: out[i] = a[i] + b[i] (b != NULL: 2 reads, 1 write),
 * out[i] = a[i] (b == NULL: 1 read, 1 write; out == a is the in-place form)
 * or out[i] = 0 (a == NULL and b == NULL: 1 write) over n floats, with the
 * elementwise kernels' memory access (non-temporal 128-bit loads and stores)
 * at a chosen launch shape: `threads` lanes per workgroup (64 or 256), `vpt`
 * float4s per lane (1, 2 or 4).  n % 4 == 0, every pointer given 16-byte
 * aligned, b only with a, and n / 4 <= 2^30, else EINVAL.  No
 * counterpart in the reference; the benchmark times it to report the
 * attainable streaming rate beside each op's. */
int fence_calib_stream(float* out, const float* a, const float* b, int64_t n, int threads, int vpt,
                       hipStream_t stream);

/* Read-only calibration stream: reads a[0, n) with the same loads and launch
 * shapes as fence_calib_stream, and wave w writes the sum of the floats it
 * read to sums[w], where lanes t of workgroup g read the float4s
 * g * threads * vpt + t + j * threads (j < vpt) and wave w = g * threads / 64
 * + t / 64: sums holds ceil(n / (4 * threads * vpt)) * threads / 64 floats.
 * n % 4 == 0, a 16-byte aligned, n / 4 <= 2^30, threads 64 or 256, vpt 1, 2
 * or 4, else EINVAL.  No counterpart in the reference; the benchmark times it
 * as the attainable rate of a GEMV's weight stream (one read, no write). */
int fence_calib_read(float* sums, const float* a, int64_t n, int threads, int vpt, hipStream_t stream);

/* Static text for a status code. */
const char* fence_status_string(int status);

/* Library version string. */
const char* fence_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FENCE_OPS_H */
