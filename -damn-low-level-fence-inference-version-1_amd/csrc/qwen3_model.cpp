// qwen3_model.cpp -- Qwen3 host forward on the gfx950 kernels (host only):
// GGUF weights to HBM, KV caches, scratch, and the per-token launch sequence
// of src/model/qwen3.cu:116-341.  Interface: include/fence/qwen3.hpp (C++),
// include/fence/model.h (C ABI).
#include "fence/model.h"
#include "fence/qwen3.hpp"

#include <hip/hip_runtime.h>
#include <sys/mman.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <new>
#include <stdexcept>
#include <thread>
#include <unordered_map>
#include <utility>

namespace {

constexpr size_t kAlign = 256;
constexpr size_t kStageBytes = size_t(64) << 20;  // one pinned staging buffer
constexpr int kCopyThreads = 4;                  // host threads filling a staging buffer
// score_buf holds kScoreBufScale x the reference's n_heads * max_ctx floats:
// room for four times as many split-sequence partials in decode attention.
constexpr int kScoreBufScale = 4;

size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// memcpy split over a few threads: the source is a file mapping whose page
// faults, not memory bandwidth, limit one thread.
void parallel_copy(void* dst, const void* src, size_t n) {
    if (n < (size_t(4) << 20)) {
        std::memcpy(dst, src, n);
        return;
    }
    std::thread th[kCopyThreads - 1];
    const size_t part = align_up((n + kCopyThreads - 1) / kCopyThreads, 4096);
    for (int i = 1; i < kCopyThreads; ++i) {
        const size_t lo = std::min(n, part * i), hi = std::min(n, part * (i + 1));
        th[i - 1] = std::thread([=] { std::memcpy(static_cast<char*>(dst) + lo, static_cast<const char*>(src) + lo, hi - lo); });
    }
    std::memcpy(dst, src, std::min(n, part));
    for (auto& t : th) t.join();
}

}  // namespace

bool Qwen3Model::fail(const std::string& why, int status) {
    error_ = why;
    status_ = status;
    return false;
}

namespace {
int hip_status(hipError_t e) { return e == hipSuccess ? FENCE_SUCCESS : FENCE_ERROR_HIP_BASE + static_cast<int>(e); }
constexpr int kUnsupported = FENCE_ERROR_UNSUPPORTED;
}  // namespace

// Config from metadata with the reference's optional keys and defaults,
// src/model/qwen3.cu:137-180.
bool Qwen3Model::read_config() {
    std::string arch = "qwen2";
    if (const GGUFMetadataKV* kv = gguf_.find_metadata("general.architecture"))
        if (kv->type == GGUFValueType::STRING) arch = std::get<std::string>(kv->value);
    try {
        config.n_layers = static_cast<int>(gguf_.get_u32(arch + ".block_count"));
        config.embed_dim = static_cast<int>(gguf_.get_u32(arch + ".embedding_length"));
        config.ff_dim = static_cast<int>(gguf_.get_u32(arch + ".feed_forward_length"));
        config.n_heads = static_cast<int>(gguf_.get_u32(arch + ".attention.head_count"));
        config.n_kv_heads = static_cast<int>(gguf_.get_u32(arch + ".attention.head_count_kv"));
    } catch (const std::exception& e) {
        return fail(e.what(), kUnsupported);
    }
    if (config.n_heads <= 0) return fail("attention.head_count must be positive", kUnsupported);
    try {
        config.head_dim = static_cast<int>(gguf_.get_u32(arch + ".attention.key_length"));
    } catch (const std::exception&) {
        config.head_dim = config.embed_dim / config.n_heads;
    }
    try {
        config.rope_freq_base = gguf_.get_f32(arch + ".rope.freq_base");
    } catch (const std::exception&) {
        config.rope_freq_base = 10000.0f;
    }
    try {
        config.rms_eps = gguf_.get_f32(arch + ".attention.layer_norm_rms_epsilon");
    } catch (const std::exception&) {
        config.rms_eps = 1e-5f;
    }
    const GGUFTensorInfo* embd = gguf_.find_tensor("token_embd.weight");
    if (!embd) return fail("missing token_embd.weight", kUnsupported);
    if (embd->n_dims != 2 || embd->dims[1] == 0 || embd->dims[1] > 0x7fffffffu)
        return fail("token_embd.weight must be a [embed_dim, vocab] matrix", kUnsupported);
    config.vocab_size = static_cast<int>(embd->dims[1]);

    const Qwen3Config& c = config;
    const int64_t dims[] = {c.n_layers, c.embed_dim, c.ff_dim, c.n_heads, c.n_kv_heads, c.head_dim};
    for (int64_t d : dims)
        if (d <= 0 || d > (1 << 24)) return fail("model dimensions must be positive and below 2^24", kUnsupported);
    if (c.n_heads % c.n_kv_heads != 0) return fail("head_count must be a multiple of head_count_kv", kUnsupported);
    if (c.head_dim % 2 != 0) return fail("head_dim must be even (RoPE pairs)", kUnsupported);
    // Q6_K rows are whole 256-weight blocks; Q8_0 rows whole 32-weight blocks
    if (c.embed_dim % 256 || c.q_dim() % 256 || c.ff_dim % 256)
        return fail("embedding_length, head_count*head_dim and feed_forward_length must be multiples of 256 (Q6_K)",
                    kUnsupported);
    return true;
}

// Lays the tensors out in one device arena.  When the file's alignment keeps
// every tensor 16-byte aligned, the arena is the file's tensor data region
// byte for byte (one contiguous copy); otherwise each tensor gets its own
// 256-byte aligned slot.
bool Qwen3Model::place_weights() {
    struct Want {
        std::string name;
        GGMLType type;
        uint32_t n_dims;
        uint64_t d0, d1;
        bool optional;
    };
    const Qwen3Config& c = config;
    std::vector<Want> want = {
        {"token_embd.weight", GGMLType::Q8_0, 2, uint64_t(c.embed_dim), uint64_t(c.vocab_size), false},
        {"output_norm.weight", GGMLType::F32, 1, uint64_t(c.embed_dim), 1, false},
    };
    for (int l = 0; l < c.n_layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        const uint64_t E = c.embed_dim, Q = c.q_dim(), KV = c.kv_dim(), FF = c.ff_dim, HD = c.head_dim;
        want.push_back({p + "attn_norm.weight", GGMLType::F32, 1, E, 1, false});
        want.push_back({p + "attn_q.weight", GGMLType::Q6_K, 2, E, Q, false});
        want.push_back({p + "attn_k.weight", GGMLType::Q6_K, 2, E, KV, false});
        want.push_back({p + "attn_v.weight", GGMLType::Q6_K, 2, E, KV, false});
        want.push_back({p + "attn_q.bias", GGMLType::F32, 1, Q, 1, true});
        want.push_back({p + "attn_k.bias", GGMLType::F32, 1, KV, 1, true});
        want.push_back({p + "attn_v.bias", GGMLType::F32, 1, KV, 1, true});
        want.push_back({p + "attn_q_norm.weight", GGMLType::F32, 1, HD, 1, true});
        want.push_back({p + "attn_k_norm.weight", GGMLType::F32, 1, HD, 1, true});
        want.push_back({p + "attn_output.weight", GGMLType::Q6_K, 2, Q, E, false});
        want.push_back({p + "ffn_norm.weight", GGMLType::F32, 1, E, 1, false});
        want.push_back({p + "ffn_gate.weight", GGMLType::Q6_K, 2, E, FF, false});
        want.push_back({p + "ffn_up.weight", GGMLType::Q6_K, 2, E, FF, false});
        want.push_back({p + "ffn_down.weight", GGMLType::Q6_K, 2, FF, E, false});
    }
    placed_.clear();
    std::vector<const GGUFTensorInfo*> found;
    for (const Want& w : want) {
        const GGUFTensorInfo* t = gguf_.find_tensor(w.name);
        if (!t) {
            if (w.optional) continue;
            return fail("missing tensor " + w.name, kUnsupported);
        }
        if (t->type != w.type)
            return fail(w.name + " is " + ggml_type_name(t->type) + ", this forward runs " + ggml_type_name(w.type),
                        kUnsupported);
        if (t->n_dims != w.n_dims || t->dims[0] != w.d0 || (w.n_dims == 2 && t->dims[1] != w.d1))
            return fail(w.name + " has a shape that does not match the config", kUnsupported);
        found.push_back(t);
    }
    // the file's own layout serves when every tensor we use sits 16-byte aligned
    // in the data region (the arena itself is 256-byte aligned)
    contiguous_ = true;
    for (const GGUFTensorInfo* t : found) contiguous_ = contiguous_ && t->offset % 16 == 0;
    size_t next = 0;
    for (const GGUFTensorInfo* t : found) {
        if (contiguous_) {
            placed_.push_back({t->name, static_cast<size_t>(t->offset), t->data_size_bytes});
        } else {
            placed_.push_back({t->name, next, t->data_size_bytes});
            next = align_up(next + t->data_size_bytes, kAlign);
        }
    }
    return true;
}

bool Qwen3Model::upload_weights() {
    struct Range {
        const uint8_t* src;
        size_t dst, bytes;
    };
    std::vector<Range> ranges;
    size_t arena = 0;
    // start of the tensor data region in the mapping (token_embd exists: checked)
    const GGUFTensorInfo* any = gguf_.find_tensor("token_embd.weight");
    const auto* base = static_cast<const uint8_t*>(any->data) - any->offset;
    if (contiguous_) {
        arena = gguf_.file_size() - gguf_.data_offset();
        ranges.push_back({base, 0, arena});
    } else {
        for (const Placed& p : placed_) {
            ranges.push_back({static_cast<const uint8_t*>(gguf_.find_tensor(p.name)->data), p.offset, p.bytes});
            arena = std::max(arena, p.offset + p.bytes);
        }
    }
    if (hipMalloc(&weight_arena_, std::max<size_t>(arena, 1)) != hipSuccess) {
        weight_arena_ = nullptr;
        return fail("out of device memory for " + std::to_string(arena) + " bytes of weights",
                    FENCE_ERROR_OUT_OF_MEMORY);
    }
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        e = hipHostMalloc(&stage[i], kStageBytes, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
    }
    bool pending[2] = {false, false};
    int slot = 0;
    for (const Range& r : ranges) {
        madvise(const_cast<uint8_t*>(r.src) - (reinterpret_cast<uintptr_t>(r.src) & 4095),
                r.bytes + (reinterpret_cast<uintptr_t>(r.src) & 4095), MADV_SEQUENTIAL);
        for (size_t o = 0; e == hipSuccess && o < r.bytes; o += kStageBytes) {
            const size_t n = std::min(kStageBytes, r.bytes - o);
            if (pending[slot]) e = hipEventSynchronize(done[slot]);
            if (e != hipSuccess) break;
            parallel_copy(stage[slot], r.src + o, n);
            e = hipMemcpyAsync(static_cast<char*>(weight_arena_) + r.dst + o, stage[slot], n, hipMemcpyHostToDevice,
                               stream_);
            if (e == hipSuccess) e = hipEventRecord(done[slot], stream_);
            pending[slot] = true;
            slot ^= 1;
        }
    }
    const hipError_t e_sync = hipStreamSynchronize(stream_);
    if (e == hipSuccess) e = e_sync;
    for (int i = 0; i < 2; ++i) {
        if (stage[i]) (void)hipHostFree(stage[i]);
        if (done[i]) (void)hipEventDestroy(done[i]);
    }
    madvise(const_cast<uint8_t*>(base) - (reinterpret_cast<uintptr_t>(base) & 4095),
            gguf_.file_size() - gguf_.data_offset() + (reinterpret_cast<uintptr_t>(base) & 4095), MADV_RANDOM);
    return e == hipSuccess ? true : fail(std::string("weight upload failed: ") + hipGetErrorString(e), hip_status(e));
}

const void* Qwen3Model::device_tensor(const std::string& name, size_t* bytes) const {
    for (const Placed& p : placed_)
        if (p.name == name) {
            if (bytes) *bytes = p.bytes;
            return static_cast<const char*>(weight_arena_) + p.offset;
        }
    return nullptr;
}

bool Qwen3Model::load(const std::string& gguf_path, int max_ctx, hipStream_t stream) {
    unload();
    error_.clear();
    status_ = FENCE_SUCCESS;
    if (max_ctx <= 0) return fail("max_ctx must be positive", FENCE_ERROR_INVALID_VALUE);
    if (!gguf_.open(gguf_path)) return fail(gguf_.last_error(), FENCE_ERROR_BAD_FILE);
    if (!read_config() || !place_weights()) {
        gguf_.close();
        return false;
    }
    config.max_ctx = max_ctx;
    if (stream) {
        stream_ = stream;
    } else {
        const hipError_t e = hipStreamCreate(&stream_);
        if (e != hipSuccess) {
            stream_ = nullptr;
            gguf_.close();
            return fail("hipStreamCreate failed", hip_status(e));
        }
        own_stream_ = true;
    }
    if (!upload_weights()) {
        const std::string why = error_;
        const int st = status_;
        unload();
        return fail(why, st);
    }
    auto dev = [&](const std::string& n) { return device_tensor(n); };
    const Qwen3Config& c = config;
    weights.token_embd = static_cast<const block_q8_0*>(dev("token_embd.weight"));
    weights.output_norm = static_cast<const float*>(dev("output_norm.weight"));
    weights.layers.assign(c.n_layers, Qwen3LayerWeights{});
    for (int l = 0; l < c.n_layers; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        Qwen3LayerWeights& w = weights.layers[l];
        auto f = [&](const char* s) { return static_cast<const float*>(dev(p + s)); };
        auto q = [&](const char* s) { return static_cast<const block_q6_K*>(dev(p + s)); };
        w.attn_norm = f("attn_norm.weight");
        w.attn_q = q("attn_q.weight");
        w.attn_k = q("attn_k.weight");
        w.attn_v = q("attn_v.weight");
        w.attn_q_bias = f("attn_q.bias");
        w.attn_k_bias = f("attn_k.bias");
        w.attn_v_bias = f("attn_v.bias");
        w.attn_q_norm = f("attn_q_norm.weight");
        w.attn_k_norm = f("attn_k_norm.weight");
        w.attn_output = q("attn_output.weight");
        w.ffn_norm = f("ffn_norm.weight");
        w.ffn_gate = q("ffn_gate.weight");
        w.ffn_up = q("ffn_up.weight");
        w.ffn_down = q("ffn_down.weight");
    }

    // KV caches: one allocation, zeroed like the reference's (src/model/qwen3.cu:50-59)
    const size_t per_cache = align_up(size_t(max_ctx) * c.kv_dim() * sizeof(__half), kAlign);
    if (hipMalloc(&kv_arena_, per_cache * 2 * c.n_layers) != hipSuccess) {
        kv_arena_ = nullptr;
        unload();
        return fail("out of device memory for the KV cache", FENCE_ERROR_OUT_OF_MEMORY);
    }
    kv_cache.k.resize(c.n_layers);
    kv_cache.v.resize(c.n_layers);
    for (int l = 0; l < c.n_layers; ++l) {
        kv_cache.k[l] = reinterpret_cast<__half*>(static_cast<char*>(kv_arena_) + per_cache * (2 * l));
        kv_cache.v[l] = reinterpret_cast<__half*>(static_cast<char*>(kv_arena_) + per_cache * (2 * l + 1));
    }

    // scratch (src/model/qwen3.cu:69-85), one allocation
    const size_t E = c.embed_dim, Q = c.q_dim(), KV = c.kv_dim(), FF = c.ff_dim;
    const size_t half_n = std::max(E, std::max(FF, Q));
    const size_t f32_sizes[] = {E, E, E, Q, KV, KV, Q, FF, FF, E, size_t(c.vocab_size),
                                size_t(kScoreBufScale) * c.n_heads * max_ctx};
    size_t total = 0;
    for (size_t n : f32_sizes) total += align_up(n * 4, kAlign);
    total += align_up(half_n * 2, kAlign) + align_up(FF * 2, kAlign) + kAlign;
    total += align_up(size_t(c.n_heads) * FENCE_ARRIVE_WORDS_PER_HEAD * 4, kAlign);
    if (hipMalloc(&scratch_arena_, total) != hipSuccess || hipHostMalloc(&host_token_, sizeof(int)) != hipSuccess) {
        unload();
        return fail("out of memory for scratch buffers", FENCE_ERROR_OUT_OF_MEMORY);
    }
    char* cur = static_cast<char*>(scratch_arena_);
    auto take = [&](size_t bytes) {
        char* p = cur;
        cur += align_up(bytes, kAlign);
        return p;
    };
    ScratchBuffers& s = scratch;
    s.hidden = reinterpret_cast<float*>(take(E * 4));
    s.residual = reinterpret_cast<float*>(take(E * 4));
    s.normed = reinterpret_cast<float*>(take(E * 4));
    s.q = reinterpret_cast<float*>(take(Q * 4));
    s.k = reinterpret_cast<float*>(take(KV * 4));
    s.v = reinterpret_cast<float*>(take(KV * 4));
    s.attn_out = reinterpret_cast<float*>(take(Q * 4));
    s.gate = reinterpret_cast<float*>(take(FF * 4));
    s.up = reinterpret_cast<float*>(take(FF * 4));
    s.down = reinterpret_cast<float*>(take(E * 4));
    s.logits = reinterpret_cast<float*>(take(size_t(c.vocab_size) * 4));
    s.score_buf = reinterpret_cast<float*>(take(size_t(kScoreBufScale) * c.n_heads * max_ctx * 4));
    s.x_half = reinterpret_cast<__half*>(take(half_n * 2));
    s.act_half = reinterpret_cast<__half*>(take(FF * 2));
    s.argmax_out = reinterpret_cast<int*>(take(sizeof(int)));
    const size_t arrive_bytes = size_t(c.n_heads) * FENCE_ARRIVE_WORDS_PER_HEAD * 4;
    attn_arrive_ = reinterpret_cast<uint32_t*>(take(arrive_bytes));
    hipError_t e = hipMemsetAsync(kv_arena_, 0, per_cache * 2 * c.n_layers, stream_);
    if (e == hipSuccess) e = hipMemsetAsync(attn_arrive_, 0, arrive_bytes, stream_);
    if (e == hipSuccess) e = hipStreamSynchronize(stream_);
    if (e != hipSuccess) {
        unload();
        return fail("clearing the KV cache failed", hip_status(e));
    }
    return true;
}

void Qwen3Model::unload() {
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (weight_arena_) (void)hipFree(weight_arena_);
    if (kv_arena_) (void)hipFree(kv_arena_);
    if (scratch_arena_) (void)hipFree(scratch_arena_);
    if (host_token_) (void)hipHostFree(host_token_);
    if (own_stream_ && stream_) (void)hipStreamDestroy(stream_);
    weight_arena_ = kv_arena_ = scratch_arena_ = nullptr;
    host_token_ = nullptr;
    attn_arrive_ = nullptr;
    stream_ = nullptr;
    own_stream_ = false;
    placed_.clear();
    weights = Qwen3Weights{};
    kv_cache = KVCache{};
    scratch = ScratchBuffers{};
    gguf_.close();
}

#define FENCE_STEP(call)                                                                             \
    do {                                                                                             \
        const int st_ = (call);                                                                      \
        if (st_ != FENCE_SUCCESS) return fail(std::string(#call) + ": " + fence_status_string(st_), st_); \
    } while (0)

// src/model/qwen3.cu:240-341, launcher for launcher.
bool Qwen3Model::forward_reference(int token_id, int pos) {
    const Qwen3Config& c = config;
    ScratchBuffers& s = scratch;
    hipStream_t st = stream_;
    const int E = c.embed_dim;
    FENCE_STEP(fence_embed_q8_0(s.hidden, weights.token_embd, token_id, E, st));
    for (int l = 0; l < c.n_layers; ++l) {
        const Qwen3LayerWeights& w = weights.layers[l];
        // forward_attention, src/model/qwen3.cu:267-313
        FENCE_STEP(hip_status(hipMemcpyAsync(s.residual, s.hidden, E * 4, hipMemcpyDeviceToDevice, st)));
        FENCE_STEP(fence_rms_norm(s.normed, s.hidden, w.attn_norm, E, c.rms_eps, st));
        FENCE_STEP(fence_f32_to_f16(s.x_half, s.normed, E, st));
        FENCE_STEP(w.attn_q_bias ? fence_gemv_q6k_bias(w.attn_q, s.x_half, w.attn_q_bias, s.q, c.q_dim(), E, st)
                                 : fence_gemv_q6k(w.attn_q, s.x_half, s.q, c.q_dim(), E, st));
        FENCE_STEP(w.attn_k_bias ? fence_gemv_q6k_bias(w.attn_k, s.x_half, w.attn_k_bias, s.k, c.kv_dim(), E, st)
                                 : fence_gemv_q6k(w.attn_k, s.x_half, s.k, c.kv_dim(), E, st));
        FENCE_STEP(w.attn_v_bias ? fence_gemv_q6k_bias(w.attn_v, s.x_half, w.attn_v_bias, s.v, c.kv_dim(), E, st)
                                 : fence_gemv_q6k(w.attn_v, s.x_half, s.v, c.kv_dim(), E, st));
        if (w.attn_q_norm && w.attn_k_norm) {
            FENCE_STEP(fence_rms_norm_per_head(s.q, w.attn_q_norm, c.n_heads, c.head_dim, c.rms_eps, st));
            FENCE_STEP(fence_rms_norm_per_head(s.k, w.attn_k_norm, c.n_kv_heads, c.head_dim, c.rms_eps, st));
        }
        FENCE_STEP(fence_apply_rope(s.q, s.k, c.head_dim, c.n_heads, c.n_kv_heads, pos, c.rope_freq_base, st));
        FENCE_STEP(fence_store_kv(kv_cache.k[l], kv_cache.v[l], s.k, s.v, pos, c.kv_dim(), c.max_ctx, st));
        FENCE_STEP(fence_gqa_attention(s.attn_out, s.q, kv_cache.k[l], kv_cache.v[l], c.head_dim, c.n_heads,
                                       c.n_kv_heads, pos + 1, c.max_ctx, s.score_buf, st));
        FENCE_STEP(fence_f32_to_f16(s.x_half, s.attn_out, c.q_dim(), st));
        FENCE_STEP(fence_gemv_q6k(w.attn_output, s.x_half, s.hidden, E, c.q_dim(), st));
        FENCE_STEP(fence_residual_add(s.hidden, s.residual, E, st));
        // forward_mlp, src/model/qwen3.cu:316-341
        FENCE_STEP(hip_status(hipMemcpyAsync(s.residual, s.hidden, E * 4, hipMemcpyDeviceToDevice, st)));
        FENCE_STEP(fence_rms_norm(s.normed, s.hidden, w.ffn_norm, E, c.rms_eps, st));
        FENCE_STEP(fence_f32_to_f16(s.x_half, s.normed, E, st));
        FENCE_STEP(fence_gemv_q6k(w.ffn_gate, s.x_half, s.gate, c.ff_dim, E, st));
        FENCE_STEP(fence_gemv_q6k(w.ffn_up, s.x_half, s.up, c.ff_dim, E, st));
        FENCE_STEP(fence_silu_elementwise_mul(s.gate, s.gate, s.up, c.ff_dim, st));
        FENCE_STEP(fence_f32_to_f16(s.x_half, s.gate, c.ff_dim, st));
        FENCE_STEP(fence_gemv_q6k(w.ffn_down, s.x_half, s.hidden, E, c.ff_dim, st));
        FENCE_STEP(fence_residual_add(s.hidden, s.residual, E, st));
    }
    FENCE_STEP(fence_rms_norm_inplace(s.hidden, weights.output_norm, E, c.rms_eps, st));
    FENCE_STEP(fence_gemv_q8_0(weights.token_embd, s.hidden, s.logits, c.vocab_size, E, st));
    return true;
}

// The same step with the sub-block outputs kept apart from the residual
// stream: each projection back to embed_dim (o, down) writes `down`, and the
// next RMSNorm adds it into the stream in the same pass (hidden + down is the
// reference's residual_add(hidden = o, residual), the same sum).  That norm
// runs inside the projection that reads it: every workgroup of the q/k/v and
// the gate/up launches normalises the row itself, and one of them writes the
// new stream row -- into the other of two buffers (hidden, residual), since the
// rest still read the old one.  q, k and v are one launch; attention applies
// QK-norm and RoPE to q itself, prepares and stores the new k and v row, and
// writes the binary16 input of the o projection; gate, up and SwiGLU are one
// launch (writing act_half).  5 calls per layer instead of 22 plus two
// copies; every result is bit-identical to the reference sequence's.
bool Qwen3Model::forward_fused(int token_id, int pos) {
    const Qwen3Config& c = config;
    ScratchBuffers& s = scratch;
    hipStream_t st = stream_;
    const int E = c.embed_dim;
    FENCE_STEP(fence_embed_q8_0(s.hidden, weights.token_embd, token_id, E, st));
    float* cur = s.hidden;           // the residual stream
    float* next = s.residual;        // receives cur + a block output
    const float* pending = nullptr;  // a block output not yet added to the stream
    for (int l = 0; l < c.n_layers; ++l) {
        const Qwen3LayerWeights& w = weights.layers[l];
        const void* w_qkv[3] = {w.attn_q, w.attn_k, w.attn_v};
        float* y_qkv[3] = {s.q, s.k, s.v};
        const float* b_qkv[3] = {w.attn_q_bias, w.attn_k_bias, w.attn_v_bias};
        const int m_qkv[3] = {c.q_dim(), c.kv_dim(), c.kv_dim()};
        const fence_rms_input attn_in{cur, pending, pending ? next : nullptr, w.attn_norm, s.x_half, c.rms_eps};
        FENCE_STEP(fence_gemv_q6k_multi_rms(3, w_qkv, y_qkv, b_qkv, m_qkv, &attn_in, E, st));
        if (pending) std::swap(cur, next);
        const bool qk_norm = w.attn_q_norm && w.attn_k_norm;
        FENCE_STEP(fence_gqa_attention_qk_f16_arrive(
            nullptr, s.x_half, s.q, s.k, s.v, qk_norm ? w.attn_q_norm : nullptr, qk_norm ? w.attn_k_norm : nullptr,
            kv_cache.k[l], kv_cache.v[l], c.head_dim, c.n_heads, c.n_kv_heads, pos, c.max_ctx, c.rms_eps,
            c.rope_freq_base, FENCE_ROPE_NEOX, s.score_buf, kScoreBufScale * int64_t(c.n_heads) * c.max_ctx,
            attn_arrive_, st));
        FENCE_STEP(fence_gemv_q6k(w.attn_output, s.x_half, s.down, E, c.q_dim(), st));
        const fence_rms_input ffn_in{cur, s.down, next, w.ffn_norm, s.x_half, c.rms_eps};
        FENCE_STEP(fence_gemv_q6k_swiglu_rms_f16(w.ffn_gate, w.ffn_up, &ffn_in, s.act_half, nullptr, c.ff_dim, E, st));
        std::swap(cur, next);
        FENCE_STEP(fence_gemv_q6k(w.ffn_down, s.act_half, s.down, E, c.ff_dim, st));
        pending = s.down;
    }
    FENCE_STEP(fence_residual_rms_norm_f16(cur, pending, weights.output_norm, s.normed, nullptr, 1, E, c.rms_eps, st));
    FENCE_STEP(fence_gemv_q8_0(weights.token_embd, s.normed, s.logits, c.vocab_size, E, st));
    return true;
}

#undef FENCE_STEP

float* Qwen3Model::forward(int token_id, int pos) {
    if (!weight_arena_) return fail("no model loaded", FENCE_ERROR_INVALID_VALUE), nullptr;
    if (token_id < 0 || token_id >= config.vocab_size)
        return fail("token " + std::to_string(token_id) + " outside [0, vocab)", FENCE_ERROR_INVALID_VALUE), nullptr;
    if (pos < 0 || pos >= config.max_ctx)
        return fail("position " + std::to_string(pos) + " outside [0, max_ctx)", FENCE_ERROR_INVALID_VALUE), nullptr;
    const bool ok = sequence_ == Qwen3Sequence::Fused ? forward_fused(token_id, pos) : forward_reference(token_id, pos);
    return ok ? scratch.logits : nullptr;
}

int Qwen3Model::sample_greedy(float* logits) {
    if (!weight_arena_ || !logits) return fail("no model loaded or no logits", FENCE_ERROR_INVALID_VALUE), -1;
    // The fused sequence reduces over many workgroups with the partials in
    // score_buf: attention's scratch, free again once this stream's forward
    // has run.  Both forms return the reference argmax's index.
    const int st = sequence_ == Qwen3Sequence::Fused
                       ? fence_argmax_ws(logits, scratch.argmax_out, config.vocab_size, scratch.score_buf,
                                         int64_t(kScoreBufScale) * config.n_heads * config.max_ctx * 4, stream_)
                       : fence_argmax(logits, scratch.argmax_out, config.vocab_size, stream_);
    if (st != FENCE_SUCCESS) return fail(std::string("argmax: ") + fence_status_string(st), st), -1;
    hipError_t e = hipMemcpyAsync(host_token_, scratch.argmax_out, sizeof(int), hipMemcpyDeviceToHost, stream_);
    if (e == hipSuccess) e = hipStreamSynchronize(stream_);
    if (e != hipSuccess) return fail("reading the argmax back failed", hip_status(e)), -1;
    return *host_token_;
}

// ------------------------------------------------------------------ C ABI

struct fence_model {
    Qwen3Model m;
};

extern "C" int fence_model_load(const char* path, int max_ctx, hipStream_t stream, fence_model** out, char* err,
                                size_t err_len) {
    if (!path || !out || max_ctx <= 0) return FENCE_ERROR_INVALID_VALUE;
    *out = nullptr;
    auto* h = new (std::nothrow) fence_model;
    if (!h) return FENCE_ERROR_OUT_OF_MEMORY;
    if (!h->m.load(path, max_ctx, stream)) {
        if (err && err_len) std::snprintf(err, err_len, "%s", h->m.error().c_str());
        const int st = h->m.last_status();
        delete h;
        return st;
    }
    *out = h;
    return FENCE_SUCCESS;
}

extern "C" void fence_model_free(fence_model* h) { delete h; }

extern "C" int fence_model_get_config(const fence_model* h, fence_model_config* out) {
    if (!h || !out) return FENCE_ERROR_INVALID_VALUE;
    const Qwen3Config& c = h->m.config;
    *out = fence_model_config{c.n_layers, c.embed_dim, c.ff_dim, c.n_heads, c.n_kv_heads, c.head_dim,
                              c.vocab_size, c.max_ctx, c.rope_freq_base, c.rms_eps, 1, 0};
    for (const Qwen3LayerWeights& w : h->m.weights.layers) {
        if (!w.attn_q_norm || !w.attn_k_norm) out->has_qk_norm = 0;
        if (w.attn_q_bias || w.attn_k_bias || w.attn_v_bias) ++out->has_qkv_bias;
    }
    return FENCE_SUCCESS;
}

extern "C" int fence_model_set_sequence(fence_model* h, int sequence) {
    if (!h || (sequence != FENCE_SEQUENCE_FUSED && sequence != FENCE_SEQUENCE_REFERENCE))
        return FENCE_ERROR_INVALID_VALUE;
    h->m.set_sequence(sequence == FENCE_SEQUENCE_FUSED ? Qwen3Sequence::Fused : Qwen3Sequence::Reference);
    return FENCE_SUCCESS;
}

extern "C" int fence_model_forward(fence_model* h, int token_id, int pos, float** logits) {
    if (!h || !logits) return FENCE_ERROR_INVALID_VALUE;
    *logits = nullptr;
    const Qwen3Config& c = h->m.config;
    if (token_id < 0 || token_id >= c.vocab_size || pos < 0 || pos >= c.max_ctx) return FENCE_ERROR_INVALID_VALUE;
    float* y = h->m.forward(token_id, pos);
    if (!y) return h->m.last_status();
    *logits = y;
    return FENCE_SUCCESS;
}

extern "C" int fence_model_sample_greedy(fence_model* h, const float* logits, int* token) {
    if (!h || !logits || !token) return FENCE_ERROR_INVALID_VALUE;
    const int t = h->m.sample_greedy(const_cast<float*>(logits));
    if (t < 0) return h->m.last_status();
    *token = t;
    return FENCE_SUCCESS;
}

extern "C" int fence_model_read_tensor(const fence_model* h, const char* name, void* dst, uint64_t capacity,
                                       uint64_t* bytes) {
    if (!h || !name) return FENCE_ERROR_INVALID_VALUE;
    size_t n = 0;
    const void* p = h->m.device_tensor(name, &n);
    if (!p) return FENCE_ERROR_NOT_FOUND;
    if (bytes) *bytes = n;
    if (!dst) return FENCE_SUCCESS;
    if (capacity < n) return FENCE_ERROR_INVALID_VALUE;
    const hipError_t e = hipMemcpy(dst, p, n, hipMemcpyDeviceToHost);
    return e == hipSuccess ? FENCE_SUCCESS : FENCE_ERROR_HIP_BASE + static_cast<int>(e);
}

extern "C" int fence_model_kv_cache(const fence_model* h, int layer, void** k_cache, void** v_cache) {
    if (!h || !k_cache || !v_cache || layer < 0 || layer >= h->m.config.n_layers ||
        layer >= static_cast<int>(h->m.kv_cache.k.size()))
        return FENCE_ERROR_INVALID_VALUE;
    *k_cache = h->m.kv_cache.k[layer];
    *v_cache = h->m.kv_cache.v[layer];
    return FENCE_SUCCESS;
}

extern "C" hipStream_t fence_model_stream(const fence_model* h) { return h ? h->m.stream() : nullptr; }
