/*
 * fence/model.h -- C ABI of the Qwen3 host forward (include/fence/qwen3.hpp)
 * for hosts that cannot use the C++ class.  Each entry point replaces a
 * member of the reference's Qwen3Model (src/model/qwen3.h:115-155).
 *
 * A model owns its device memory (weights, KV caches, scratch) and, when the
 * caller passes a null stream, a stream of its own.  Calls on one model are
 * not thread-safe; different models are independent.
 */
#ifndef FENCE_MODEL_H
#define FENCE_MODEL_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "fence/ops.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct fence_model fence_model;

/* Qwen3Config, src/model/qwen3.h:19-44, as read from the file; plus which
 * optional tensors the file has. */
typedef struct {
    int n_layers, embed_dim, ff_dim, n_heads, n_kv_heads, head_dim, vocab_size, max_ctx;
    float rope_freq_base, rms_eps;
    int has_qk_norm;  /* every layer has attn_q_norm and attn_k_norm */
    int has_qkv_bias; /* number of layers with at least one q/k/v bias */
} fence_model_config;

/* Which kernel sequence forward launches. */
enum {
    FENCE_SEQUENCE_FUSED = 0,     /* q/k/v in one launch that also computes its input
                                     norm, gate/up + SwiGLU (and its norm) in another;
                                     QK-norm + RoPE + KV store inside attention */
    FENCE_SEQUENCE_REFERENCE = 1  /* the launch order of src/model/qwen3.cu:267-341 */
};

/* Qwen3Model::load, src/model/qwen3.h:123 (src/model/qwen3.cu:116-230), on
 * the current device.  max_ctx > 0 (the reference's default is 4096).
 * Returns FENCE_ERROR_BAD_FILE, FENCE_ERROR_UNSUPPORTED (a tensor missing or
 * of another type or shape), FENCE_ERROR_OUT_OF_MEMORY or a HIP error; err
 * (may be NULL) receives the reason. */
int fence_model_load(const char* gguf_path, int max_ctx, hipStream_t stream, fence_model** out,
                     char* err, size_t err_len);
/* Qwen3Model::unload and delete, src/model/qwen3.h:124. */
void fence_model_free(fence_model* m);

int fence_model_get_config(const fence_model* m, fence_model_config* out);
int fence_model_set_sequence(fence_model* m, int sequence);

/* Qwen3Model::forward, src/model/qwen3.h:131 (src/model/qwen3.cu:240-341):
 * one token at position pos, enqueued on the model's stream; *logits = the
 * device logits [vocab_size] (valid until the next forward).  EINVAL for a
 * token outside [0, vocab) or pos outside [0, max_ctx). */
int fence_model_forward(fence_model* m, int token_id, int pos, float** logits);

/* Qwen3Model::sample_greedy, src/model/qwen3.h:134: argmax of device logits
 * [vocab_size] (the first index of the maximum); synchronises the stream. */
int fence_model_sample_greedy(fence_model* m, const float* logits, int* token);

/* Copies the device copy of file tensor `name` into host memory (capacity
 * bytes at dst); *bytes = its size.  NOT_FOUND if the model did not load it,
 * EINVAL if capacity is too small.  Synchronous. */
int fence_model_read_tensor(const fence_model* m, const char* name, void* dst, uint64_t capacity,
                            uint64_t* bytes);

/* Device pointers of layer l's binary16 KV caches [max_ctx][kv_dim]. */
int fence_model_kv_cache(const fence_model* m, int layer, void** k_cache, void** v_cache);

/* The model's stream. */
hipStream_t fence_model_stream(const fence_model* m);

#ifdef __cplusplus
}
#endif

#endif /* FENCE_MODEL_H */
