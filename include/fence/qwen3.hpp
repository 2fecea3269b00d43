/*
 * fence/qwen3.hpp -- the host forward of a Qwen3 decode step on the gfx950
 * kernels, with the reference's model interface (src/model/qwen3.h:19-155):
 * Qwen3Config, Qwen3LayerWeights, Qwen3Weights, KVCache, ScratchBuffers and
 * Qwen3Model with load / unload / forward / sample_greedy.
 *
 * Differences from the reference, all on the side of failing loudly:
 *   - load() checks every tensor's presence, type and shape against the
 *     config (the reference copies a missing tensor as a null pointer and
 *     would fault later) and reports why in error();
 *   - forward() rejects a token outside [0, vocab) or a position outside
 *     [0, max_ctx) and returns nullptr (the reference reads or writes out of
 *     bounds);
 *   - forward() is asynchronous on the model's stream (the reference
 *     synchronises the device after each stage); sample_greedy synchronises.
 * Memory: the weights live in one device allocation (each tensor 256-byte
 * aligned), the KV caches in a second, the scratch buffers in a third.
 * Sampling other than greedy and the generation loop (src/model/qwen3.cu:
 * 350-519) are host code outside this library.
 */
#ifndef FENCE_QWEN3_HPP
#define FENCE_QWEN3_HPP

#include <cstdint>
#include <string>
#include <vector>

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include "fence/gguf_parser.hpp"
#include "fence/q6k_types.h"
#include "fence/q8_0_types.h"

/* src/model/qwen3.h:19-44 (the sampling fields belong to the host's sampler) */
struct Qwen3Config {
    int n_layers = 36;
    int embed_dim = 2560;
    int ff_dim = 9728;
    int n_heads = 32;
    int n_kv_heads = 8;
    int head_dim = 128;
    int vocab_size = 151936;
    int max_ctx = 4096;
    float rope_freq_base = 5000000.0f;
    float rms_eps = 1e-6f;

    int q_dim() const { return n_heads * head_dim; }
    int kv_dim() const { return n_kv_heads * head_dim; }
    int heads_per_group() const { return n_heads / n_kv_heads; }
};

/* src/model/qwen3.h:47-65; optional tensors (biases, QK-norm) are null when
 * the file has none. */
struct Qwen3LayerWeights {
    const float* attn_norm = nullptr;
    const block_q6_K* attn_q = nullptr;
    const block_q6_K* attn_k = nullptr;
    const block_q6_K* attn_v = nullptr;
    const float* attn_q_bias = nullptr;
    const float* attn_k_bias = nullptr;
    const float* attn_v_bias = nullptr;
    const float* attn_q_norm = nullptr;
    const float* attn_k_norm = nullptr;
    const block_q6_K* attn_output = nullptr;
    const float* ffn_norm = nullptr;
    const block_q6_K* ffn_gate = nullptr;
    const block_q6_K* ffn_up = nullptr;
    const block_q6_K* ffn_down = nullptr;
};

/* src/model/qwen3.h:68-76: token_embd is also the (tied) LM head. */
struct Qwen3Weights {
    const block_q8_0* token_embd = nullptr;
    const float* output_norm = nullptr;
    std::vector<Qwen3LayerWeights> layers;
};

/* src/model/qwen3.h:79-88: per-layer binary16 caches [max_ctx][kv_dim]. */
struct KVCache {
    std::vector<__half*> k;
    std::vector<__half*> v;
};

/* src/model/qwen3.h:91-112 (cpu_logits is the host sampler's). */
struct ScratchBuffers {
    float* hidden = nullptr;     // [embed_dim]
    float* residual = nullptr;   // [embed_dim]: the reference sequence's copy; the fused one's second stream row
    float* normed = nullptr;     // [embed_dim]
    float* q = nullptr;          // [q_dim]
    float* k = nullptr;          // [kv_dim]
    float* v = nullptr;          // [kv_dim]
    float* attn_out = nullptr;   // [q_dim]
    float* gate = nullptr;       // [ff_dim]
    float* up = nullptr;         // [ff_dim]
    float* down = nullptr;       // [embed_dim]
    float* logits = nullptr;     // [vocab_size]
    float* score_buf = nullptr;  // [4 * n_heads * max_ctx]: attention's split-sequence partials
    __half* x_half = nullptr;    // [max(embed_dim, ff_dim, q_dim)]
    int* argmax_out = nullptr;   // [1]
    __half* act_half = nullptr;  // [ff_dim]: SwiGLU output of the fused sequence
};

/* The kernel sequence forward() launches. */
enum class Qwen3Sequence {
    Fused,      // layer-boundary norms inside the q/k/v and gate/up launches, q/k/v, QK-norm +
                // RoPE + KV store inside attention (+ conversion), gate/up + SwiGLU: 6 calls per layer
    Reference,  // the reference's launcher order, src/model/qwen3.cu:267-341
};

/* src/model/qwen3.h:115-155 */
class Qwen3Model {
public:
    Qwen3Config config;
    Qwen3Weights weights;
    KVCache kv_cache;
    ScratchBuffers scratch;

    Qwen3Model() = default;
    ~Qwen3Model() { unload(); }
    Qwen3Model(const Qwen3Model&) = delete;
    Qwen3Model& operator=(const Qwen3Model&) = delete;

    /* src/model/qwen3.h:123: read the GGUF file, copy the weights to the
     * current device, allocate the KV cache and scratch.  max_ctx as in the
     * reference's Qwen3Config (4096); stream null = a stream of the model's
     * own (default priority). */
    bool load(const std::string& gguf_path) { return load(gguf_path, 4096, nullptr); }
    bool load(const std::string& gguf_path, int max_ctx, hipStream_t stream);
    void unload();

    /* src/model/qwen3.h:131: one token at position pos; the KV caches keep
     * positions 0..pos.  Returns the device logits [vocab_size], or nullptr
     * (see error()). */
    float* forward(int token_id, int pos);

    /* src/model/qwen3.h:134: argmax of device logits [vocab_size]; -1 on error. */
    int sample_greedy(float* logits);

    void set_sequence(Qwen3Sequence s) { sequence_ = s; }
    Qwen3Sequence sequence() const { return sequence_; }
    hipStream_t stream() const { return stream_; }
    const std::string& error() const { return error_; }
    /* Status of the last failure (a FENCE_ERROR_* code, include/fence/ops.h). */
    int last_status() const { return status_; }
    const GGUFFile& gguf() const { return gguf_; }
    /* Device copy of a file tensor by GGUF name (nullptr if not loaded). */
    const void* device_tensor(const std::string& name, size_t* bytes = nullptr) const;

private:
    GGUFFile gguf_;
    void* weight_arena_ = nullptr;
    void* kv_arena_ = nullptr;
    void* scratch_arena_ = nullptr;
    int* host_token_ = nullptr;  // pinned
    uint32_t* attn_arrive_ = nullptr;  // the one-launch attention's counters, zero between calls
    hipStream_t stream_ = nullptr;
    bool own_stream_ = false;
    Qwen3Sequence sequence_ = Qwen3Sequence::Fused;
    std::string error_;
    int status_ = 0;
    bool contiguous_ = false;  // the arena is the file's tensor data region
    struct Placed {
        std::string name;
        size_t offset, bytes;
    };
    std::vector<Placed> placed_;

    bool fail(const std::string& why, int status);
    bool read_config();
    bool place_weights();
    bool upload_weights();
    bool forward_fused(int token_id, int pos);
    bool forward_reference(int token_id, int pos);
};

#endif /* FENCE_QWEN3_HPP */
