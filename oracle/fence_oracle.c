/*
 * fence_oracle.c -- scalar CPU restatement of Fence's fused per-layer ops.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels, never part of
 * the product path.  Build: see oracle/Makefile (gcc -O2 -ffp-contract=off,
 * no fast-math).  Numerics conventions are stated in fence_oracle.h.
 */
#include "fence_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static float bits_to_f32(uint32_t b) {
    float f;
    memcpy(&f, &b, sizeof f);
    return f;
}

static uint32_t f32_to_bits(float f) {
    uint32_t b;
    memcpy(&b, &f, sizeof b);
    return b;
}

/* IEEE binary16 -> binary32, exact for every finite input.
 * The reference decodes with __half2float (src/kernels/gemv_q8_0.cuh:27). */
float fo_fp16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    if (exp == 0) {
        if (man == 0) return bits_to_f32(sign);
        /* subnormal: man * 2^-24, exactly representable in fp32 */
        const float mag = (float)man * 0x1p-24f;
        return bits_to_f32(sign | f32_to_bits(mag));
    }
    if (exp == 31) {
        uint32_t b = sign | 0x7F800000u | (man << 13);
        if (man) b |= 0x00400000u; /* quiet the NaN */
        return bits_to_f32(b);
    }
    return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* ---------------------------------------------------------------- RMSNorm */

/* src/kernels/ops.cuh:17-45: ss = sum x^2; r = rsqrt(ss/n + eps);
 * out[i] = w[i] * x[i] * r, multiplied in that order. */
static float rms_scale(const float* x, int n, float eps) {
    double ss = 0.0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * (double)x[i];
    return (float)(1.0 / sqrt(ss / (double)n + (double)eps));
}

void fo_rms_norm(float* out, const float* x, const float* w, int n, float eps) {
    const float r = rms_scale(x, n, eps);
    for (int i = 0; i < n; ++i) out[i] = (w[i] * x[i]) * r;
}

/* src/kernels/ops.cuh:54-60 */
void fo_rms_norm_inplace(float* x, const float* w, int n, float eps) {
    fo_rms_norm(x, x, w, n, eps);
}

void fo_rms_norm_rows(float* out, const float* x, const float* w,
                      int64_t rows, int n, float eps) {
    for (int64_t r = 0; r < rows; ++r)
        fo_rms_norm(out + r * n, x + r * n, w, n, eps);
}

/* src/kernels/ops.cuh:66-95: each head of head_dim values normalised on its
 * own, the weight w[head_dim] shared by all heads. */
void fo_rms_norm_per_head(float* x, const float* w, int n_heads, int head_dim,
                          float eps) {
    for (int h = 0; h < n_heads; ++h) {
        float* hx = x + (int64_t)h * head_dim;
        fo_rms_norm(hx, hx, w, head_dim, eps);
    }
}

/* ------------------------------------------------------------------- RoPE */

/* src/kernels/ops.cuh:133: freq = 1.0f / powf(base, (float)(2p) / (float)hd) */
void fo_rope_inv_freq(float* inv_freq, int head_dim, float freq_base) {
    for (int p = 0; p < head_dim / 2; ++p)
        inv_freq[p] = 1.0f / powf(freq_base, (float)(2 * p) / (float)head_dim);
}

/* src/kernels/ops.cuh:133-144 (NeoX: pair (p, p+hd/2)) and the interleaved
 * form of its comment, ops.cuh:109-113 (pair (2p, 2p+1)):
 *   a = (float)pos * freq;  x0' = x0 cos a - x1 sin a;  x1' = x0 sin a + x1 cos a */
void fo_rope_head(float* x, int head_dim, int pos, float freq_base, int style) {
    const int half = head_dim / 2;
    for (int p = 0; p < half; ++p) {
        const float freq = 1.0f / powf(freq_base, (float)(2 * p) / (float)head_dim);
        const float angle = (float)pos * freq;
        const float c = cosf(angle);
        const float s = sinf(angle);
        const int i0 = (style == FO_ROPE_NEOX) ? p : 2 * p;
        const int i1 = (style == FO_ROPE_NEOX) ? p + half : 2 * p + 1;
        const float x0 = x[i0];
        const float x1 = x[i1];
        x[i0] = x0 * c - x1 * s;
        x[i1] = x0 * s + x1 * c;
    }
}

/* src/kernels/ops.cuh:115-177: all q heads, then all k heads, one position */
void fo_apply_rope(float* q, float* k, int head_dim, int n_q_heads,
                   int n_kv_heads, int pos, float freq_base) {
    for (int h = 0; h < n_q_heads; ++h)
        fo_rope_head(q + (int64_t)h * head_dim, head_dim, pos, freq_base, FO_ROPE_NEOX);
    for (int h = 0; h < n_kv_heads; ++h)
        fo_rope_head(k + (int64_t)h * head_dim, head_dim, pos, freq_base, FO_ROPE_NEOX);
}

static int token_pos(const int32_t* positions, int pos0, int64_t t) {
    return positions ? positions[t] : pos0 + (int)t;
}

void fo_rope_rows(float* q, float* k, int64_t tokens, int n_q_heads,
                  int n_kv_heads, int head_dim, const int32_t* positions,
                  int pos0, float freq_base, int style) {
    const int64_t qrow = (int64_t)n_q_heads * head_dim;
    const int64_t krow = (int64_t)n_kv_heads * head_dim;
    for (int64_t t = 0; t < tokens; ++t) {
        const int pos = token_pos(positions, pos0, t);
        for (int h = 0; h < n_q_heads; ++h)
            fo_rope_head(q + t * qrow + (int64_t)h * head_dim, head_dim, pos,
                         freq_base, style);
        if (k)
            for (int h = 0; h < n_kv_heads; ++h)
                fo_rope_head(k + t * krow + (int64_t)h * head_dim, head_dim, pos,
                             freq_base, style);
    }
}

/* ----------------------------------------------------------------- SwiGLU */

/* src/kernels/ops.cuh:189-194: out = (g / (1 + expf(-g))) * up */
void fo_silu_elementwise_mul(float* out, const float* gate, const float* up,
                             int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        const float g = gate[i];
        const float silu_g = g / (1.0f + expf(-g));
        out[i] = silu_g * up[i];
    }
}

/* ---------------------------------------------------------------- softmax */

/* src/kernels/ops.cuh:207-246 (and the decode form ops.cuh:357-391):
 * m = max(-1e30f, x_i); e_i = expf(x_i - m); x_i = e_i * (1.0f / sum e). */
static void softmax_row(float* x, int n_valid) {
    float m = -1e30f;
    for (int i = 0; i < n_valid; ++i) m = fmaxf(m, x[i]);
    double s = 0.0;
    for (int i = 0; i < n_valid; ++i) {
        const float e = expf(x[i] - m);
        x[i] = e;
        s += (double)e;
    }
    const float inv = 1.0f / (float)s;
    for (int i = 0; i < n_valid; ++i) x[i] *= inv;
}

void fo_softmax(float* x, int n) { softmax_row(x, n); }

void fo_softmax_rows(float* x, int64_t rows, int n, int64_t ld) {
    for (int64_t r = 0; r < rows; ++r) softmax_row(x + r * ld, n);
}

void fo_softmax_causal(float* x, int64_t heads, int sq, int sk) {
    for (int64_t h = 0; h < heads; ++h) {
        for (int i = 0; i < sq; ++i) {
            float* row = x + (h * sq + i) * (int64_t)sk;
            int valid = i + 1 + (sk - sq);
            if (valid < 0) valid = 0;
            if (valid > sk) valid = sk;
            softmax_row(row, valid);
            for (int j = valid; j < sk; ++j) row[j] = 0.0f;
        }
    }
}

/* ------------------------------------------------------------------- Q8_0 */

/* the fp16 scale d of a block, stored little-endian in its first two bytes */
static float block_scale(const uint8_t* blk) {
    return fo_fp16_to_f32((uint16_t)(blk[0] | ((uint16_t)blk[1] << 8)));
}

/* src/kernels/gemv_q8_0.cuh:12-29 with the block layout of
 * src/kernels/q8_0_types.h:10-15: out[i] = half2float(d[i/32]) * qs[i/32][i%32] */
void fo_embed_q8_0(float* out, const uint8_t* table, int token_id, int dim) {
    const int nb = dim / FO_QK8_0;
    const uint8_t* row = table + (int64_t)token_id * nb * FO_Q8_0_BLOCK_BYTES;
    for (int i = 0; i < dim; ++i) {
        const uint8_t* blk = row + (i / FO_QK8_0) * FO_Q8_0_BLOCK_BYTES;
        const float d = block_scale(blk);
        const int8_t q = (int8_t)blk[2 + i % FO_QK8_0];
        out[i] = d * (float)q;
    }
}

int64_t fo_embed_q8_0_gather(float* out, const uint8_t* table, int64_t vocab,
                             const int32_t* ids, int64_t tokens, int dim) {
    int64_t bad = 0;
    for (int64_t t = 0; t < tokens; ++t) {
        float* o = out + t * dim;
        if (ids[t] < 0 || ids[t] >= vocab) {
            for (int i = 0; i < dim; ++i) o[i] = bits_to_f32(0x7FC00000u);
            ++bad;
            continue;
        }
        fo_embed_q8_0(o, table, ids[t], dim);
    }
    return bad;
}

int64_t fo_embed_q8_0_gather_rms_norm(float* out, const uint8_t* table,
                                      int64_t vocab, const int32_t* ids,
                                      int64_t tokens, int dim, const float* w,
                                      float eps) {
    const int64_t bad = fo_embed_q8_0_gather(out, table, vocab, ids, tokens, dim);
    for (int64_t t = 0; t < tokens; ++t) {
        float* o = out + t * dim;
        fo_rms_norm(o, o, w, dim, eps);
    }
    return bad;
}

/* src/kernels/gemv_q8_0.cuh:40-60 (q8_0_dot_f32_warp_partial) and :75-97:
 * y[row] = sum_b d_b * (sum_i qs[b][i] * x[32b + i]); the reference sums in
 * fp32 per lane then across the warp; the oracle accumulates in double. */
void fo_gemv_q8_0(const uint8_t* W, const float* x, float* y, int M, int K) {
    const int nb = K / FO_QK8_0;
    for (int r = 0; r < M; ++r) {
        const uint8_t* row = W + (int64_t)r * nb * FO_Q8_0_BLOCK_BYTES;
        double sum = 0.0;
        for (int b = 0; b < nb; ++b) {
            const uint8_t* blk = row + b * FO_Q8_0_BLOCK_BYTES;
            const double d = block_scale(blk);
            double block_sum = 0.0;
            for (int i = 0; i < FO_QK8_0; ++i)
                block_sum += (double)(int8_t)blk[2 + i] * (double)x[b * FO_QK8_0 + i];
            sum += d * block_sum;
        }
        y[r] = (float)sum;
    }
}

/* ------------------------------------------------------------------- Q6_K */

/* src/kernels/q6k_dot.cuh:35-64: element i of a block sits in half i/128,
 * column (i%128)/32, lane l = i%32: its low nibble is ql[64*half + l (+32 for
 * columns 1 and 3)], the low or high nibble (columns 0-1 / 2-3); its two high
 * bits are bits 2*column of qh[32*half + l]. */
int fo_q6k_quant(const uint8_t* blk, int i) {
    const int half = i / 128, col = (i % 128) / 32, l = i % 32;
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int lo = (ql[64 * half + l + ((col & 1) ? 32 : 0)] >> ((col >= 2) ? 4 : 0)) & 0xF;
    const int hi = (qh[32 * half + l] >> (2 * col)) & 0x3;
    return lo | (hi << 4);
}

double fo_q6k_dot(const uint8_t* blk, const uint16_t* x16) {
    const int8_t* scales = (const int8_t*)(blk + 192);
    const double d = fo_fp16_to_f32((uint16_t)(blk[208] | ((uint16_t)blk[209] << 8)));
    double sum = 0.0;
    for (int i = 0; i < FO_QK_K; ++i)
        sum += d * (double)scales[i / 16] * (double)(fo_q6k_quant(blk, i) - 32) *
               (double)fo_fp16_to_f32(x16[i]);
    return sum;
}

/* src/kernels/gemv_q6k.cuh:44-84 (and :107-138 with the bias) */
void fo_gemv_q6k(const uint8_t* W, const uint16_t* x16, const float* bias, float* y,
                 int M, int K) {
    const int nb = K / FO_QK_K;
    for (int r = 0; r < M; ++r) {
        double sum = 0.0;
        for (int b = 0; b < nb; ++b)
            sum += fo_q6k_dot(W + ((int64_t)r * nb + b) * FO_Q6K_BLOCK_BYTES, x16 + b * FO_QK_K);
        y[r] = bias ? (float)sum + bias[r] : (float)sum;
    }
}

/* ------------------------------------------------- f16 and residual epilogue */

/* src/kernels/ops.cuh:448-462 (f32_to_f16) and :274-289 (float_to_half):
 * out[i] = __float2half(in[i]), IEEE round to nearest even. */
uint16_t fo_f32_to_f16(float f) {
    const uint32_t b = f32_to_bits(f);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const uint32_t exp = (b >> 23) & 0xFFu;
    const uint32_t man = b & 0x7FFFFFu;
    if (exp == 0xFFu) /* inf, or NaN made quiet */
        return (uint16_t)(sign | 0x7C00u | (man ? 0x0200u | (man >> 13) : 0u));
    if (exp >= 113u) { /* normal in binary16 unless rounding carries past 65504 */
        const uint32_t e16 = exp - 112u;
        if (e16 >= 31u) return (uint16_t)(sign | 0x7C00u);
        uint32_t h = (e16 << 10) | (man >> 13);
        const uint32_t rem = man & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* a carry may reach inf */
        return (uint16_t)(sign | h);
    }
    /* binary16 subnormal or zero: value = sig * 2^(exp-150), unit 2^-24 */
    const uint32_t shift = 126u - exp; /* >= 14 */
    if (exp == 0u || shift > 24u) return (uint16_t)sign;
    const uint32_t sig = man | 0x800000u;
    uint32_t q = sig >> shift;
    const uint32_t rem = sig & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
}

void fo_f32_to_f16_array(uint16_t* out, const float* in, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = fo_f32_to_f16(in[i]);
}

/* src/kernels/ops.cuh:256-270 */
void fo_residual_add(float* x, const float* residual, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] += residual[i];
}

/* src/model/qwen3.cu:312 then :318-325 (residual_add; rms_norm; f32_to_f16) */
void fo_residual_rms_norm_f16(float* hidden, const float* residual, const float* w,
                              float* normed, uint16_t* out16, int64_t rows, int n,
                              float eps) {
    for (int64_t r = 0; r < rows; ++r) {
        float* h = hidden + r * n;
        if (residual) fo_residual_add(h, residual + r * n, n);
        const float rs = rms_scale(h, n, eps);
        for (int i = 0; i < n; ++i) {
            const float v = (w[i] * h[i]) * rs;
            if (normed) normed[r * n + i] = v;
            if (out16) out16[r * n + i] = fo_f32_to_f16(v);
        }
    }
}

/* src/model/qwen3.cu:332-336 (silu_elementwise_mul; f32_to_f16) */
void fo_swiglu_f16(uint16_t* out16, float* out, const float* gate, const float* up,
                   int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        float v;
        fo_silu_elementwise_mul(&v, gate + i, up + i, 1);
        if (out) out[i] = v;
        out16[i] = fo_f32_to_f16(v);
    }
}

/* ------------------------------------------------- decode attention, KV */

/* src/kernels/ops.cuh:419-432 */
void fo_store_kv(uint16_t* k_cache, uint16_t* v_cache, const float* k, const float* v,
                 int pos, int kv_dim) {
    for (int i = 0; i < kv_dim; ++i) {
        k_cache[(int64_t)pos * kv_dim + i] = fo_f32_to_f16(k[i]);
        v_cache[(int64_t)pos * kv_dim + i] = fo_f32_to_f16(v[i]);
    }
}

/* src/kernels/ops.cuh:320-404 */
void fo_gqa_attention(float* out, const float* q, const uint16_t* k_cache,
                      const uint16_t* v_cache, int head_dim, int n_q_heads,
                      int n_kv_heads, int seq_len, int max_ctx) {
    (void)max_ctx;
    const int group = n_q_heads / n_kv_heads;
    const int64_t kv_dim = (int64_t)n_kv_heads * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float s_small[1];
    float* s = seq_len > 0 ? (float*)malloc(sizeof(float) * (size_t)seq_len) : s_small;
    for (int h = 0; h < n_q_heads; ++h) {
        const int kvh = h / group;
        const float* qh = q + (int64_t)h * head_dim;
        for (int t = 0; t < seq_len; ++t) {
            const uint16_t* kt = k_cache + t * kv_dim + (int64_t)kvh * head_dim;
            double dot = 0.0;
            for (int d = 0; d < head_dim; ++d) dot += (double)qh[d] * (double)fo_fp16_to_f32(kt[d]);
            s[t] = (float)dot * scale;
        }
        softmax_row(s, seq_len);
        for (int d = 0; d < head_dim; ++d) {
            double acc = 0.0;
            for (int t = 0; t < seq_len; ++t)
                acc += (double)s[t] * (double)fo_fp16_to_f32(v_cache[t * kv_dim + (int64_t)kvh * head_dim + d]);
            out[(int64_t)h * head_dim + d] = (float)acc;
        }
    }
    if (s != s_small) free(s);
}

/* argmax, src/kernels/ops.cuh:467-505: the reference's one 256-thread block.
 * Ties follow its tree, not the lowest index: among the threads t = i mod 256
 * holding the maximum, the one with the smallest 8-bit bit-reversal of t wins
 * (maxima at 1 and 256 give 256, at 1 and 2 give 2); within a thread, the
 * first index. */
int fo_argmax(const float* x, int n) {
    /* src/kernels/ops.cuh:476-485, 256 threads (:502): thread t scans x[t],
     * x[t+256], .. keeping the first value strictly above its maximum. */
    enum { THREADS = 256 };
    float sv[THREADS];
    int si[THREADS];
    for (int t = 0; t < THREADS; ++t) {
        float local_max = -1e30f;
        int local_idx = 0;
        for (int i = t; i < n; i += THREADS)
            if (x[i] > local_max) {
                local_max = x[i];
                local_idx = i;
            }
        sv[t] = local_max;
        si[t] = local_idx;
    }
    /* ops.cuh:488-498: slot u takes slot u+s only if strictly greater. */
    for (int s = THREADS / 2; s > 0; s >>= 1)
        for (int u = 0; u < s; ++u)
            if (sv[u + s] > sv[u]) {
                sv[u] = sv[u + s];
                si[u] = si[u + s];
            }
    return si[0];
}

/* ------------------------------------------------------ fused compositions */

void fo_qk_norm_rope(float* q, float* k, const float* wq, const float* wk,
                     int64_t tokens, int n_q_heads, int n_kv_heads,
                     int head_dim, float eps, const int32_t* positions,
                     int pos0, float freq_base, int style) {
    const int64_t qrow = (int64_t)n_q_heads * head_dim;
    const int64_t krow = (int64_t)n_kv_heads * head_dim;
    for (int64_t t = 0; t < tokens; ++t) {
        fo_rms_norm_per_head(q + t * qrow, wq, n_q_heads, head_dim, eps);
        if (k) fo_rms_norm_per_head(k + t * krow, wk, n_kv_heads, head_dim, eps);
    }
    fo_rope_rows(q, k, tokens, n_q_heads, n_kv_heads, head_dim, positions, pos0,
                 freq_base, style);
}

void fo_rms_norm_rope(float* out, const float* x, const float* w, float* k,
                      int64_t tokens, int n_q_heads, int n_kv_heads,
                      int head_dim, float eps, const int32_t* positions,
                      int pos0, float freq_base, int style) {
    const int n = n_q_heads * head_dim;
    fo_rms_norm_rows(out, x, w, tokens, n, eps);
    fo_rope_rows(out, k, tokens, n_q_heads, n_kv_heads, head_dim, positions, pos0,
                 freq_base, style);
}
