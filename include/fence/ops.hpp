/*
 * fence/ops.hpp -- drop-in launchers with the reference's names, argument
 * order and defaults (src/kernels/ops.cuh, src/kernels/gemv_q8_0.cuh), so a
 * HIP build of the reference's model code (src/model/qwen3.cu) calls the
 * gfx950 kernels without changing a call site: include this header where it
 * included ops.cuh / gemv_q8_0.cuh.
 *
 * Like the reference launchers these return void.  The status of the last
 * call on this host thread is kept for fence_last_status(); an invalid
 * argument launches nothing (the reference launchers would have launched
 * anyway and failed later, at the next synchronisation).
 */
#ifndef FENCE_OPS_HPP
#define FENCE_OPS_HPP

#include "fence/ops.h"
#include "fence/q6k_types.h"
#include "fence/q8_0_types.h"

namespace fence_detail {
inline int& last_status() {
    thread_local int status = FENCE_SUCCESS;
    return status;
}
inline void record(int status) { last_status() = status; }
}  // namespace fence_detail

/* Status of the most recent launcher call on this thread (0 = success). */
inline int fence_last_status() { return fence_detail::last_status(); }

/* src/kernels/ops.cuh:47 */
inline void rms_norm(float* out, const float* x, const float* w, int n, float eps,
                     hipStream_t stream = 0) {
    fence_detail::record(fence_rms_norm(out, x, w, n, eps, stream));
}

/* src/kernels/ops.cuh:54 */
inline void rms_norm_inplace(float* x, const float* w, int n, float eps, hipStream_t stream = 0) {
    fence_detail::record(fence_rms_norm_inplace(x, w, n, eps, stream));
}

/* src/kernels/ops.cuh:97 */
inline void rms_norm_per_head(float* x, const float* w, int n_heads, int head_dim, float eps,
                              hipStream_t stream = 0) {
    fence_detail::record(fence_rms_norm_per_head(x, w, n_heads, head_dim, eps, stream));
}

/* src/kernels/ops.cuh:169 */
inline void apply_rope(float* q, float* k, int head_dim, int n_q_heads, int n_kv_heads, int pos,
                       float freq_base, hipStream_t stream = 0) {
    fence_detail::record(
        fence_apply_rope(q, k, head_dim, n_q_heads, n_kv_heads, pos, freq_base, stream));
}

/* src/kernels/ops.cuh:197 */
inline void silu_elementwise_mul(float* out, const float* gate, const float* up, int n,
                                 hipStream_t stream = 0) {
    fence_detail::record(fence_silu_elementwise_mul(out, gate, up, n, stream));
}

/* src/kernels/ops.cuh:248 */
inline void softmax(float* x, int n, hipStream_t stream = 0) {
    fence_detail::record(fence_softmax(x, n, stream));
}

/* src/kernels/gemv_q8_0.cuh:31 */
inline void embed_q8_0(float* d_out, const block_q8_0* d_weight, int token_id, int dim,
                       hipStream_t stream = 0) {
    fence_detail::record(fence_embed_q8_0(d_out, d_weight, token_id, dim, stream));
}

/* src/kernels/gemv_q8_0.cuh:99 */
inline void gemv_q8_0(const block_q8_0* d_W, const float* d_x, float* d_y, int M, int K,
                      hipStream_t stream = 0) {
    fence_detail::record(fence_gemv_q8_0(d_W, d_x, d_y, M, K, stream));
}

/* src/kernels/gemv_q6k.cuh:89 */
inline void gemv_q6k(const block_q6_K* d_W, const __half* d_x, float* d_y, int M, int K,
                     hipStream_t stream = 0) {
    fence_detail::record(fence_gemv_q6k(d_W, d_x, d_y, M, K, stream));
}

/* src/kernels/gemv_q6k.cuh:140 */
inline void gemv_q6k_bias(const block_q6_K* d_W, const __half* d_x, const float* d_bias, float* d_y,
                          int M, int K, hipStream_t stream = 0) {
    fence_detail::record(fence_gemv_q6k_bias(d_W, d_x, d_bias, d_y, M, K, stream));
}

/* src/kernels/ops.cuh:405 */
inline void gqa_attention(float* attn_out, const float* q, const half* k_cache, const half* v_cache,
                          int head_dim, int n_q_heads, int n_kv_heads, int seq_len, int max_ctx,
                          float* score_buf, hipStream_t stream = 0) {
    fence_detail::record(fence_gqa_attention(attn_out, q, k_cache, v_cache, head_dim, n_q_heads,
                                             n_kv_heads, seq_len, max_ctx, score_buf, stream));
}

/* src/kernels/ops.cuh:435 */
inline void store_kv(half* k_cache, half* v_cache, const float* k, const float* v, int pos,
                     int kv_dim, int max_ctx, hipStream_t stream = 0) {
    fence_detail::record(fence_store_kv(k_cache, v_cache, k, v, pos, kv_dim, max_ctx, stream));
}

/* src/kernels/ops.cuh:501 */
inline void argmax(const float* x, int* result, int n, hipStream_t stream = 0) {
    fence_detail::record(fence_argmax(x, result, n, stream));
}

/* src/kernels/ops.cuh:265 */
inline void residual_add(float* x, const float* residual, int n, hipStream_t stream = 0) {
    fence_detail::record(fence_residual_add(x, residual, n, stream));
}

/* src/kernels/ops.cuh:457 */
inline void f32_to_f16(half* out, const float* in, int n, hipStream_t stream = 0) {
    fence_detail::record(fence_f32_to_f16(out, in, n, stream));
}

/* src/kernels/ops.cuh:284 */
inline void float_to_half(half* out, const float* in, int n, hipStream_t stream = 0) {
    fence_detail::record(fence_f32_to_f16(out, in, n, stream));
}

/* src/kernels/ops.cuh:303 */
inline void half_to_float(float* out, const half* in, int n, hipStream_t stream = 0) {
    fence_detail::record(fence_f16_to_f32(out, in, n, stream));
}

#endif /* FENCE_OPS_HPP */
