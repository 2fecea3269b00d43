// decode_step.cpp -- a whole Qwen3-4B-shaped decode step through this
// library, in the order of src/model/qwen3.cu:246-341 (forward,
// forward_attention, forward_mlp), on synthetic weights.
//
//   decode_step            check mode: one layer and the LM head through the
//                          reference's launcher names (include/fence/ops.hpp);
//                          every stage is compared with the oracle, fed the
//                          device's own output of the stage before.  Prints one
//                          PASS/FAIL line per check; exit status = failures.
//   decode_step --time [L] [pos] [--no-graph]
//                          L layers (default 36) of distinct synthetic Q6_K
//                          weights and KV caches filled up to pos (default
//                          2915) on the device; prints one JSON line with the
//                          microseconds per token of (a) the reference's launch
//                          sequence, (b) the fused entry points, (c) (b)
//                          replayed as one HIP graph per token.
#include "fence/ops.hpp"
#include "fence_oracle.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#define HIP_CHECK(call)                                                                    \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess) {                                                            \
            std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, \
                         __LINE__);                                                        \
            std::exit(100);                                                                \
        }                                                                                  \
    } while (0)

namespace {

// Qwen3-4B (src/model/qwen3.h:19-44), rope base of BASELINE configs[0]
constexpr int E = 2560, FF = 9728, NQ = 32, NKV = 8, HD = 128, V = 151936, CTX = 4096;
constexpr int QD = NQ * HD, KVD = NKV * HD;
constexpr float EPS = 1e-6f, BASE = 1e6f;

// ------------------------------------------------------------ device fill

__device__ __forceinline__ uint32_t mix(uint64_t x) {
    x ^= x >> 33;
    x *= 0xFF51AFD7ED558CCDull;
    x ^= x >> 33;
    x *= 0xC4CEB9FE1A85EC53ull;
    x ^= x >> 33;
    return static_cast<uint32_t>(x);
}

// Q6_K blocks: random ql/qh, scales uniform in [-8, 7], d fixed (binary16 bits).
__global__ void fill_q6k(uint8_t* w, int64_t nblocks, uint64_t seed, uint16_t d_bits) {
    const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    uint8_t* blk = w + b * 210;
    for (int i = 0; i < 192; i += 4) {
        const uint32_t r = mix(seed ^ (static_cast<uint64_t>(b) << 8) ^ static_cast<uint64_t>(i));
        blk[i] = r & 0xFF, blk[i + 1] = (r >> 8) & 0xFF, blk[i + 2] = (r >> 16) & 0xFF, blk[i + 3] = r >> 24;
    }
    for (int i = 0; i < 16; ++i)
        blk[192 + i] = static_cast<uint8_t>(static_cast<int8_t>((mix(seed * 3 + b * 16 + i) & 15) - 8));
    blk[208] = d_bits & 0xFF;
    blk[209] = d_bits >> 8;
}

// binary16 values ~ uniform in [-1, 1)
__global__ void fill_f16(uint16_t* p, int64_t n, uint64_t seed) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>((mix(seed ^ i) >> 8) * (2.0f / 16777216.0f) - 1.0f));
}

// Q8_0 table: d = 2^-12, int8 uniform
__global__ void fill_q8(uint8_t* t, int64_t nblocks, uint64_t seed) {
    const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= nblocks) return;
    uint8_t* blk = t + b * 34;
    blk[0] = 0x00, blk[1] = 0x0C;  // 2^-12
    for (int i = 0; i < 32; i += 4) {
        const uint32_t r = mix(seed ^ (static_cast<uint64_t>(b) << 6) ^ i);
        blk[2 + i] = r & 0xFF, blk[3 + i] = (r >> 8) & 0xFF, blk[4 + i] = (r >> 16) & 0xFF, blk[5 + i] = r >> 24;
    }
}

unsigned blocks_for(int64_t n) { return static_cast<unsigned>((n + 255) / 256); }

template <class T>
T* dalloc(size_t n) {
    T* p = nullptr;
    HIP_CHECK(hipMalloc(&p, n * sizeof(T)));
    return p;
}

struct Layer {
    float *attn_norm, *q_norm, *k_norm, *ffn_norm;
    uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;  // Q6_K
    uint16_t *kc, *vc;                         // KV cache, binary16 [CTX][KVD]
};

int64_t q6_bytes(int m, int k) { return static_cast<int64_t>(m) * (k / 256) * 210; }

void fill_layer(Layer& L, uint64_t seed, std::vector<float>* norms_out = nullptr) {
    const uint16_t d = 0x1400;  // binary16 2^-10
    struct W {
        uint8_t** p;
        int m, k;
    } ws[] = {{&L.wq, QD, E}, {&L.wk, KVD, E}, {&L.wv, KVD, E}, {&L.wo, E, QD},
              {&L.wg, FF, E}, {&L.wu, FF, E}, {&L.wd, E, FF}};
    int i = 0;
    for (auto& w : ws) {
        *w.p = dalloc<uint8_t>(q6_bytes(w.m, w.k));
        const int64_t nb = q6_bytes(w.m, w.k) / 210;
        fill_q6k<<<blocks_for(nb), 256>>>(*w.p, nb, seed * 131 + i++, d);
    }
    L.kc = dalloc<uint16_t>(static_cast<size_t>(CTX) * KVD);
    L.vc = dalloc<uint16_t>(static_cast<size_t>(CTX) * KVD);
    fill_f16<<<blocks_for(static_cast<int64_t>(CTX) * KVD), 256>>>(L.kc, static_cast<int64_t>(CTX) * KVD, seed * 7 + 1);
    fill_f16<<<blocks_for(static_cast<int64_t>(CTX) * KVD), 256>>>(L.vc, static_cast<int64_t>(CTX) * KVD, seed * 7 + 2);
    std::vector<float> nw(E * 2 + HD * 2);
    uint64_t s = seed;
    for (auto& x : nw) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        x = 1.0f + 0.1f * ((s >> 40) * (2.0f / 16777216.0f) - 1.0f);
    }
    L.attn_norm = dalloc<float>(E), L.ffn_norm = dalloc<float>(E), L.q_norm = dalloc<float>(HD),
    L.k_norm = dalloc<float>(HD);
    HIP_CHECK(hipMemcpy(L.attn_norm, nw.data(), E * 4, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(L.ffn_norm, nw.data() + E, E * 4, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(L.q_norm, nw.data() + 2 * E, HD * 4, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(L.k_norm, nw.data() + 2 * E + HD, HD * 4, hipMemcpyHostToDevice));
    if (norms_out) *norms_out = nw;
}

void free_layer(Layer& L) {
    for (void* p : {static_cast<void*>(L.attn_norm), static_cast<void*>(L.q_norm), static_cast<void*>(L.k_norm),
                    static_cast<void*>(L.ffn_norm), static_cast<void*>(L.wq), static_cast<void*>(L.wk),
                    static_cast<void*>(L.wv), static_cast<void*>(L.wo), static_cast<void*>(L.wg),
                    static_cast<void*>(L.wu), static_cast<void*>(L.wd), static_cast<void*>(L.kc),
                    static_cast<void*>(L.vc)})
        (void)hipFree(p);
}

struct Scratch {  // the reference's ScratchBuffers (src/model/qwen3.h:91-112)
    float *hidden, *residual, *normed, *q, *k, *v, *attn_out, *gate, *up, *tmp, *logits, *score_buf;
    half* x_half;
    half* act_half;  // SwiGLU output of the fused sequence (x_half is its input)
    int* argmax_out;
    uint32_t* arrive;  // attention's arrival counters (zeroed once; every call leaves them zero)
    void alloc() {
        hidden = dalloc<float>(E), residual = dalloc<float>(E), normed = dalloc<float>(E), q = dalloc<float>(QD),
        k = dalloc<float>(KVD), v = dalloc<float>(KVD), attn_out = dalloc<float>(QD), gate = dalloc<float>(FF),
        up = dalloc<float>(FF), tmp = dalloc<float>(E), logits = dalloc<float>(V),
        score_buf = dalloc<float>(4 * static_cast<size_t>(NQ) * CTX);  // 4x: more attention splits
        x_half = dalloc<half>(FF);
        act_half = dalloc<half>(FF);
        argmax_out = dalloc<int>(1);
        arrive = dalloc<uint32_t>(NQ * FENCE_ARRIVE_WORDS_PER_HEAD);
        HIP_CHECK(hipMemset(arrive, 0, NQ * FENCE_ARRIVE_WORDS_PER_HEAD * sizeof(uint32_t)));
    }
};

// ------------------------------------------------------------ one layer

// The reference's launch sequence, src/model/qwen3.cu:267-341.
void layer_reference(const Layer& L, Scratch& s, int pos, hipStream_t st) {
    HIP_CHECK(hipMemcpyAsync(s.residual, s.hidden, E * 4, hipMemcpyDeviceToDevice, st));
    rms_norm(s.normed, s.hidden, L.attn_norm, E, EPS, st);
    f32_to_f16(s.x_half, s.normed, E, st);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wq), s.x_half, s.q, QD, E, st);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wk), s.x_half, s.k, KVD, E, st);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wv), s.x_half, s.v, KVD, E, st);
    rms_norm_per_head(s.q, L.q_norm, NQ, HD, EPS, st);
    rms_norm_per_head(s.k, L.k_norm, NKV, HD, EPS, st);
    apply_rope(s.q, s.k, HD, NQ, NKV, pos, BASE, st);
    store_kv(reinterpret_cast<half*>(L.kc), reinterpret_cast<half*>(L.vc), s.k, s.v, pos, KVD, CTX, st);
    gqa_attention(s.attn_out, s.q, reinterpret_cast<half*>(L.kc), reinterpret_cast<half*>(L.vc), HD, NQ, NKV,
                  pos + 1, CTX, s.score_buf, st);
    f32_to_f16(s.x_half, s.attn_out, QD, st);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wo), s.x_half, s.hidden, E, QD, st);
    residual_add(s.hidden, s.residual, E, st);
    HIP_CHECK(hipMemcpyAsync(s.residual, s.hidden, E * 4, hipMemcpyDeviceToDevice, st));
    rms_norm(s.normed, s.hidden, L.ffn_norm, E, EPS, st);
    f32_to_f16(s.x_half, s.normed, E, st);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wg), s.x_half, s.gate, FF, E, st);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wu), s.x_half, s.up, FF, E, st);
    silu_elementwise_mul(s.gate, s.gate, s.up, FF, st);
    f32_to_f16(s.x_half, s.gate, FF, st);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wd), s.x_half, s.hidden, E, FF, st);
    residual_add(s.hidden, s.residual, E, st);
}

// The same layer through the fused entry points.  On entry s.tmp holds the
// previous block's output still to be added to s.hidden (zeros before the
// first layer); on exit s.tmp holds this layer's down projection.  The
// layer-boundary norms run inside the q/k/v and gate/up launches, which write
// hidden + tmp into s.residual (their workgroups still read s.hidden); the two
// pointers then swap, so s.hidden is always the stream -- and after a whole
// layer (two swaps) the same buffer again.
void layer_fused(const Layer& L, Scratch& s, int pos, hipStream_t st) {
    const void* w_qkv[3] = {L.wq, L.wk, L.wv};
    float* y_qkv[3] = {s.q, s.k, s.v};
    const int m_qkv[3] = {QD, KVD, KVD};
    const fence_rms_input attn_in{s.hidden, s.tmp, s.residual, L.attn_norm, s.x_half, EPS};
    fence_gemv_q6k_multi_rms(3, w_qkv, y_qkv, nullptr, m_qkv, &attn_in, E, st);
    std::swap(s.hidden, s.residual);
    fence_gqa_attention_qk_f16_arrive(nullptr, s.x_half, s.q, s.k, s.v, L.q_norm, L.k_norm, L.kc, L.vc, HD, NQ, NKV,
                                      pos, CTX, EPS, BASE, FENCE_ROPE_NEOX, s.score_buf, 4 * int64_t(NQ) * CTX,
                                      s.arrive, st);
    fence_gemv_q6k(L.wo, s.x_half, s.tmp, E, QD, st);
    const fence_rms_input ffn_in{s.hidden, s.tmp, s.residual, L.ffn_norm, s.x_half, EPS};
    fence_gemv_q6k_swiglu_rms_f16(L.wg, L.wu, &ffn_in, s.act_half, nullptr, FF, E, st);
    std::swap(s.hidden, s.residual);
    fence_gemv_q6k(L.wd, s.act_half, s.tmp, E, FF, st);
}

// ------------------------------------------------------------ check mode

int g_pass = 0, g_fail = 0;

void report(const char* name, bool ok, double worst) {
    std::printf("%s %-46s worst %.3e\n", ok ? "PASS" : "FAIL", name, worst);
    (ok ? g_pass : g_fail)++;
}

template <class T>
std::vector<T> get(const T* d, size_t n) {
    std::vector<T> h(n);
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
    return h;
}

// per row of `row`: max|got-ref| <= 1e-5 max|ref|
void rows_close(const char* name, const std::vector<float>& got, const std::vector<float>& ref, int row) {
    double worst = 0;
    bool ok = got.size() == ref.size();
    for (size_t r0 = 0; ok && r0 < ref.size(); r0 += row) {
        double d = 0, m = 0;
        for (int i = 0; i < row; ++i) {
            d = std::fmax(d, std::fabs((double)got[r0 + i] - ref[r0 + i]));
            m = std::fmax(m, std::fabs((double)ref[r0 + i]));
        }
        if (!(d <= 1e-5 * m)) ok = false;
        worst = std::fmax(worst, m > 0 ? d / m : d);
    }
    report(name, ok, worst);
}

template <class T>
void bits_equal(const char* name, const std::vector<T>& got, const std::vector<T>& ref) {
    report(name, got.size() == ref.size() && std::memcmp(got.data(), ref.data(), got.size() * sizeof(T)) == 0, 0);
}

// GEMV bar: per row |y - y_ref| <= 1e-5 * sum_j |W_rj x_j|
void gemv_close(const char* name, const uint8_t* Wq6, const std::vector<uint16_t>& x16, const std::vector<float>& got,
                int M, int K) {
    std::vector<float> ref(M);
    fo_gemv_q6k(Wq6, x16.data(), nullptr, ref.data(), M, K);
    std::vector<double> ax(K);
    for (int j = 0; j < K; ++j) ax[j] = std::fabs(fo_fp16_to_f32(x16[j]));
    double worst = 0;
    bool ok = true;
    const int nb = K / 256;
    for (int r = 0; r < M; ++r) {
        double scale = 0;
        for (int b = 0; b < nb; ++b) {
            const uint8_t* blk = Wq6 + (static_cast<int64_t>(r) * nb + b) * 210;
            const double d = std::fabs(fo_fp16_to_f32(static_cast<uint16_t>(blk[208] | (blk[209] << 8))));
            for (int i = 0; i < 256; ++i)
                scale += d * std::abs(static_cast<int8_t>(blk[192 + i / 16])) *
                         std::abs(fo_q6k_quant(blk, i) - 32) * ax[256 * b + i];
        }
        const double err = std::fabs((double)got[r] - ref[r]);
        if (!(err <= 1e-5 * scale)) ok = false;
        worst = std::fmax(worst, scale > 0 ? err / scale : err);
    }
    report(name, ok, worst);
}

int check_mode() {
    const int pos = 100, token = 9707;
    Layer L{};
    std::vector<float> nw;
    fill_layer(L, 11, &nw);
    const float* w_attn = nw.data();
    const float* w_ffn = nw.data() + E;
    const float* w_q = nw.data() + 2 * E;
    const float* w_k = nw.data() + 2 * E + HD;
    uint8_t* table = dalloc<uint8_t>(static_cast<size_t>(V) * (E / 32) * 34);
    fill_q8<<<blocks_for(static_cast<int64_t>(V) * (E / 32)), 256>>>(table, static_cast<int64_t>(V) * (E / 32), 5);
    float* out_norm = dalloc<float>(E);
    HIP_CHECK(hipMemcpy(out_norm, w_attn, E * 4, hipMemcpyHostToDevice));
    Scratch s;
    s.alloc();
    auto host_bytes = [](const uint8_t* d, int64_t n) { return get(d, n); };
    const auto hq = host_bytes(L.wq, q6_bytes(QD, E)), hk = host_bytes(L.wk, q6_bytes(KVD, E)),
               hv = host_bytes(L.wv, q6_bytes(KVD, E)), ho = host_bytes(L.wo, q6_bytes(E, QD)),
               hg = host_bytes(L.wg, q6_bytes(FF, E)), hu = host_bytes(L.wu, q6_bytes(FF, E)),
               hd = host_bytes(L.wd, q6_bytes(E, FF));
    const auto htab = host_bytes(table, static_cast<int64_t>(V) * (E / 32) * 34);

    // forward (qwen3.cu:246): embed
    embed_q8_0(s.hidden, reinterpret_cast<const block_q8_0*>(table), token, E);
    std::vector<float> h(E);
    fo_embed_q8_0(h.data(), htab.data(), token, E);
    bits_equal("embed_q8_0", get(s.hidden, E), h);

    // forward_attention (qwen3.cu:267-313), stage by stage
    HIP_CHECK(hipMemcpy(s.residual, s.hidden, E * 4, hipMemcpyDeviceToDevice));
    rms_norm(s.normed, s.hidden, L.attn_norm, E, EPS);
    std::vector<float> n_ref(E);
    fo_rms_norm(n_ref.data(), h.data(), w_attn, E, EPS);
    const auto dn = get(s.normed, E);
    rows_close("rms_norm(attn)", dn, n_ref, E);
    f32_to_f16(s.x_half, s.normed, E);
    std::vector<uint16_t> x16(E);
    fo_f32_to_f16_array(x16.data(), dn.data(), E);
    const auto dx = get(reinterpret_cast<uint16_t*>(s.x_half), E);
    bits_equal("f32_to_f16(normed)", dx, x16);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wq), s.x_half, s.q, QD, E);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wk), s.x_half, s.k, KVD, E);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wv), s.x_half, s.v, KVD, E);
    auto dq = get(s.q, QD), dk = get(s.k, KVD), dvv = get(s.v, KVD);
    gemv_close("gemv_q6k q 4096x2560", hq.data(), dx, dq, QD, E);
    gemv_close("gemv_q6k k 1024x2560", hk.data(), dx, dk, KVD, E);
    gemv_close("gemv_q6k v 1024x2560", hv.data(), dx, dvv, KVD, E);
    rms_norm_per_head(s.q, L.q_norm, NQ, HD, EPS);
    rms_norm_per_head(s.k, L.k_norm, NKV, HD, EPS);
    fo_rms_norm_per_head(dq.data(), w_q, NQ, HD, EPS);
    fo_rms_norm_per_head(dk.data(), w_k, NKV, HD, EPS);
    auto dq2 = get(s.q, QD), dk2 = get(s.k, KVD);
    rows_close("rms_norm_per_head(q)", dq2, dq, HD);
    rows_close("rms_norm_per_head(k)", dk2, dk, HD);
    apply_rope(s.q, s.k, HD, NQ, NKV, pos, BASE);
    fo_apply_rope(dq2.data(), dk2.data(), HD, NQ, NKV, pos, BASE);
    const auto dq3 = get(s.q, QD), dk3 = get(s.k, KVD);
    rows_close("apply_rope(q)", dq3, dq2, HD);
    rows_close("apply_rope(k)", dk3, dk2, HD);
    auto kc = get(L.kc, static_cast<size_t>(CTX) * KVD), vc = get(L.vc, static_cast<size_t>(CTX) * KVD);
    store_kv(reinterpret_cast<half*>(L.kc), reinterpret_cast<half*>(L.vc), s.k, s.v, pos, KVD, CTX);
    fo_store_kv(kc.data(), vc.data(), dk3.data(), dvv.data(), pos, KVD);
    const auto kc2 = get(L.kc, static_cast<size_t>(CTX) * KVD), vc2 = get(L.vc, static_cast<size_t>(CTX) * KVD);
    bits_equal("store_kv (k cache)", kc2, kc);
    bits_equal("store_kv (v cache)", vc2, vc);
    gqa_attention(s.attn_out, s.q, reinterpret_cast<half*>(L.kc), reinterpret_cast<half*>(L.vc), HD, NQ, NKV, pos + 1,
                  CTX, s.score_buf);
    {
        std::vector<float> ref(QD);
        fo_gqa_attention(ref.data(), dq3.data(), kc2.data(), vc2.data(), HD, NQ, NKV, pos + 1, CTX);
        const auto got = get(s.attn_out, QD);
        double vmax = 0;  // the bar's scale: the largest attended |v|
        for (int t = 0; t <= pos; ++t)
            for (int i = 0; i < KVD; ++i) vmax = std::fmax(vmax, std::fabs(fo_fp16_to_f32(vc2[(size_t)t * KVD + i])));
        double worst = 0;
        for (int i = 0; i < QD; ++i) worst = std::fmax(worst, std::fabs((double)got[i] - ref[i]));
        report("gqa_attention (err / max|v|)", worst <= 1e-5 * vmax, worst / vmax);
    }
    f32_to_f16(s.x_half, s.attn_out, QD);
    const auto dxa = get(reinterpret_cast<uint16_t*>(s.x_half), QD);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wo), s.x_half, s.hidden, E, QD);
    const auto dhid = get(s.hidden, E);
    gemv_close("gemv_q6k o 2560x4096", ho.data(), dxa, dhid, E, QD);
    residual_add(s.hidden, s.residual, E);
    std::vector<float> h2(dhid);
    fo_residual_add(h2.data(), h.data(), E);
    const auto dh2 = get(s.hidden, E);
    bits_equal("residual_add (attention)", dh2, h2);

    // forward_mlp (qwen3.cu:316-341)
    HIP_CHECK(hipMemcpy(s.residual, s.hidden, E * 4, hipMemcpyDeviceToDevice));
    rms_norm(s.normed, s.hidden, L.ffn_norm, E, EPS);
    fo_rms_norm(n_ref.data(), dh2.data(), w_ffn, E, EPS);
    const auto dn2 = get(s.normed, E);
    rows_close("rms_norm(ffn)", dn2, n_ref, E);
    f32_to_f16(s.x_half, s.normed, E);
    const auto dx2 = get(reinterpret_cast<uint16_t*>(s.x_half), E);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wg), s.x_half, s.gate, FF, E);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wu), s.x_half, s.up, FF, E);
    auto dgate = get(s.gate, FF), dup = get(s.up, FF);
    gemv_close("gemv_q6k gate 9728x2560", hg.data(), dx2, dgate, FF, E);
    gemv_close("gemv_q6k up 9728x2560", hu.data(), dx2, dup, FF, E);
    silu_elementwise_mul(s.gate, s.gate, s.up, FF);
    fo_silu_elementwise_mul(dgate.data(), dgate.data(), dup.data(), FF);
    const auto dact = get(s.gate, FF);
    rows_close("silu_elementwise_mul", dact, dgate, FF);
    f32_to_f16(s.x_half, s.gate, FF);
    const auto dx3 = get(reinterpret_cast<uint16_t*>(s.x_half), FF);
    gemv_q6k(reinterpret_cast<const block_q6_K*>(L.wd), s.x_half, s.hidden, E, FF);
    const auto ddown = get(s.hidden, E);
    gemv_close("gemv_q6k down 2560x9728", hd.data(), dx3, ddown, E, FF);
    residual_add(s.hidden, s.residual, E);
    std::vector<float> h3(ddown);
    fo_residual_add(h3.data(), dh2.data(), E);
    const auto dh3 = get(s.hidden, E);
    bits_equal("residual_add (mlp)", dh3, h3);

    // the same layer through the fused entry points ends at the same hidden state
    {
        HIP_CHECK(hipMemcpy(s.hidden, h.data(), E * 4, hipMemcpyHostToDevice));
        HIP_CHECK(hipMemset(s.tmp, 0, E * 4));
        // the caches as the reference sequence left them; the fused layer
        // overwrites row pos with its own k and v
        HIP_CHECK(hipMemcpy(L.kc, kc.data(), kc.size() * 2, hipMemcpyHostToDevice));
        HIP_CHECK(hipMemcpy(L.vc, vc.data(), vc.size() * 2, hipMemcpyHostToDevice));
        layer_fused(L, s, pos, nullptr);
        fence_residual_add(s.hidden, s.tmp, E, nullptr);
        // every fused kernel rounds as the chain it replaces: the same bits
        bits_equal("fused layer, bit for bit the reference sequence", get(s.hidden, E), dh3);
        bits_equal("fused layer, same k/v cache rows", get(L.kc, kc2.size()), kc2);
    }

    // final norm and tied LM head (qwen3.cu:257-261), greedy token
    HIP_CHECK(hipMemcpy(s.hidden, dh3.data(), E * 4, hipMemcpyHostToDevice));
    rms_norm_inplace(s.hidden, out_norm, E, EPS);
    std::vector<float> fin(dh3);
    fo_rms_norm_inplace(fin.data(), w_attn, E, EPS);
    const auto dfin = get(s.hidden, E);
    rows_close("rms_norm_inplace(output)", dfin, fin, E);
    gemv_q8_0(reinterpret_cast<const block_q8_0*>(table), s.hidden, s.logits, V, E);
    const auto dl = get(s.logits, V);
    {
        std::vector<float> ref(V);
        fo_gemv_q8_0(htab.data(), dfin.data(), ref.data(), V, E);
        double worst = 0;
        bool ok = true;
        for (int r = 0; r < V; ++r) {
            double scale = 0;
            for (int b = 0; b < E / 32; ++b) {
                const uint8_t* blk = htab.data() + (static_cast<int64_t>(r) * (E / 32) + b) * 34;
                const double dd = std::fabs(fo_fp16_to_f32(static_cast<uint16_t>(blk[0] | (blk[1] << 8))));
                for (int i = 0; i < 32; ++i)
                    scale += dd * std::abs(static_cast<int8_t>(blk[2 + i])) * std::fabs(dfin[32 * b + i]);
            }
            const double err = std::fabs((double)dl[r] - ref[r]);
            if (!(err <= 1e-5 * scale)) ok = false;
            worst = std::fmax(worst, scale > 0 ? err / scale : err);
        }
        report("gemv_q8_0 LM head (err / sum|wx|)", ok, worst);
    }
    argmax(s.logits, s.argmax_out, V);
    const auto tok = get(s.argmax_out, 1);
    report("argmax(logits)", tok[0] == fo_argmax(dl.data(), V), 0);
    fence_argmax_ws(s.logits, s.argmax_out, V, s.score_buf, 16 * int64_t(NQ) * CTX, nullptr);
    const auto tok_ws = get(s.argmax_out, 1);
    report("argmax over many workgroups (fence_argmax_ws)", tok_ws[0] == tok[0], 0);

    std::printf("%d/%d passed\n", g_pass, g_pass + g_fail);
    free_layer(L);
    return g_fail;
}

// ------------------------------------------------------------ time mode

// reps: timed tokens of each sequence (after 3 warm-up tokens);
// fused_only: skip the reference launch order (about 4x the dispatches of
// the fused one), for profiler passes that serialise every dispatch.
int time_mode(int n_layers, int pos, bool with_graph, int reps, bool fused_only) {
    std::vector<Layer> layers(n_layers);
    for (int l = 0; l < n_layers; ++l) fill_layer(layers[l], 100 + l);
    uint8_t* table = dalloc<uint8_t>(static_cast<size_t>(V) * (E / 32) * 34);
    fill_q8<<<blocks_for(static_cast<int64_t>(V) * (E / 32)), 256>>>(table, static_cast<int64_t>(V) * (E / 32), 5);
    float* out_norm = dalloc<float>(E);
    std::vector<float> ones(E, 1.0f);
    HIP_CHECK(hipMemcpy(out_norm, ones.data(), E * 4, hipMemcpyHostToDevice));
    Scratch s;
    s.alloc();
    hipStream_t st;
    HIP_CHECK(hipStreamCreate(&st));
    HIP_CHECK(hipDeviceSynchronize());

    auto token_reference = [&](int token) {
        embed_q8_0(s.hidden, reinterpret_cast<const block_q8_0*>(table), token, E, st);
        for (auto& L : layers) layer_reference(L, s, pos, st);
        rms_norm_inplace(s.hidden, out_norm, E, EPS, st);
        gemv_q8_0(reinterpret_cast<const block_q8_0*>(table), s.hidden, s.logits, V, E, st);
        argmax(s.logits, s.argmax_out, V, st);
    };
    auto token_fused = [&](int token) {
        fence_embed_q8_0(s.hidden, table, token, E, st);
        HIP_CHECK(hipMemsetAsync(s.tmp, 0, E * 4, st));
        for (auto& L : layers) layer_fused(L, s, pos, st);
        fence_residual_rms_norm_f16(s.hidden, s.tmp, out_norm, s.normed, s.x_half, 1, E, EPS, st);
        fence_gemv_q8_0(table, s.normed, s.logits, V, E, st);
        fence_argmax_ws(s.logits, s.argmax_out, V, s.score_buf, 16 * int64_t(NQ) * CTX, st);
    };
    hipEvent_t e0, e1;
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    auto time_it = [&](auto&& step, int warm, int reps) {
        for (int i = 0; i < warm; ++i) step(i);
        HIP_CHECK(hipStreamSynchronize(st));
        HIP_CHECK(hipEventRecord(e0, st));
        for (int i = 0; i < reps; ++i) step(i);
        HIP_CHECK(hipEventRecord(e1, st));
        HIP_CHECK(hipEventSynchronize(e1));
        float ms = 0;
        HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
        return 1e3 * ms / reps;
    };
    const double us_ref = fused_only ? 0.0 : time_it(token_reference, 3, reps);
    const double us_fused = time_it(token_fused, 3, reps);
    // (c) one token of (b) captured as a graph (its memset becomes a copy from
    // a zeroed buffer)
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    double us_graph = 0.0;
    float* zeros = dalloc<float>(E);
    if (with_graph) {
    HIP_CHECK(hipMemset(zeros, 0, E * 4));
    HIP_CHECK(hipDeviceSynchronize());
    HIP_CHECK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
    fence_embed_q8_0(s.hidden, table, 9707, E, st);
    HIP_CHECK(hipMemcpyAsync(s.tmp, zeros, E * 4, hipMemcpyDeviceToDevice, st));
    for (auto& L : layers) layer_fused(L, s, pos, st);
    fence_residual_rms_norm_f16(s.hidden, s.tmp, out_norm, s.normed, s.x_half, 1, E, EPS, st);
    fence_gemv_q8_0(table, s.normed, s.logits, V, E, st);
    fence_argmax_ws(s.logits, s.argmax_out, V, s.score_buf, 16 * int64_t(NQ) * CTX, st);
    HIP_CHECK(hipStreamEndCapture(st, &graph));
    HIP_CHECK(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0));
    us_graph = time_it([&](int) { HIP_CHECK(hipGraphLaunch(exec, st)); }, 3, reps);
    }

    const double weight_bytes = n_layers * (double)(q6_bytes(QD, E) + 2 * q6_bytes(KVD, E) + q6_bytes(E, QD) +
                                                    2 * q6_bytes(FF, E) + q6_bytes(E, FF)) +
                                (double)V * (E / 32) * 34;
    const double kv_bytes = n_layers * 2.0 * (pos + 1) * KVD * 2;
    std::printf("{\"layers\": %d, \"pos\": %d, \"us_per_token_reference_sequence\": %.1f, "
                "\"us_per_token_fused\": %.1f, \"us_per_token_fused_graph\": %.1f, "
                "\"weight_bytes_per_token\": %.0f, \"kv_bytes_per_token\": %.0f, "
                "\"GBps_fused_graph\": %.1f}\n",
                n_layers, pos, us_ref, us_fused, us_graph, weight_bytes, kv_bytes,
                (weight_bytes + kv_bytes) / ((with_graph ? us_graph : us_fused) * 1e-6) / 1e9);
    if (with_graph) {
        HIP_CHECK(hipGraphExecDestroy(exec));
        HIP_CHECK(hipGraphDestroy(graph));
    }
    for (auto& L : layers) free_layer(L);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc >= 2 && std::string(argv[1]) == "--time") {
        // --time [layers] [pos] [--no-graph] [--fused-only] [--tokens N]
        int layers = 36, pos = 2915, reps = 10, npos = 0;
        bool graph = true, fused_only = false, bad = false;
        for (int i = 2; i < argc; ++i) {
            const std::string a = argv[i];
            if (a == "--no-graph") graph = false;
            else if (a == "--fused-only") fused_only = true;
            else if (a == "--tokens" && i + 1 < argc) reps = std::atoi(argv[++i]);
            else if (npos == 0 && !a.empty() && a[0] != '-') layers = std::atoi(argv[i]), ++npos;
            else if (npos == 1 && !a.empty() && a[0] != '-') pos = std::atoi(argv[i]), ++npos;
            else bad = true;
        }
        if (bad || layers < 1 || layers > 64 || pos < 0 || pos >= CTX || reps < 1 || reps > 1000) {
            std::fprintf(stderr,
                         "usage: decode_step [--time [layers 1..64] [pos 0..%d] [--no-graph] [--fused-only] "
                         "[--tokens 1..1000]]\n", CTX - 1);
            return 2;
        }
        return time_mode(layers, pos, graph, reps, fused_only);
    }
    return check_mode();
}
