// attention.hip -- decode-step attention over the binary16 KV cache, and the
// KV store, on gfx950.
//
// Follows gqa_attention, src/kernels/ops.cuh:320-413: for query head h (kv
// head h / (n_q/n_kv)), over the seq_len cached positions t,
//   s_t = (q_h . k_t) * scale,   p = softmax(s),   out_h = sum_t p_t v_t,
// with caches laid out [max_ctx][n_kv][head_dim] in binary16 and
// scale = 1/sqrt(head_dim) (computed on the host, rounded to fp32).  And
// store_kv, ops.cuh:419-443: k_cache[pos][i] = binary16(k[i]), v likewise.
//
// The reference runs one 256-thread block per query head (32 blocks for
// Qwen3-4B on a 256-CU GPU) and reads each kv head's K and V once per query
// head of its group.  Here the sequence is split over many workgroups
// (split-K decoding): a workgroup takes one kv head, GT query heads of its
// group and one range of positions, so K and V rows are read once for the
// whole group.  16 lanes per position (8 dims each, one 128-bit load of K and
// one of V per lane); the q . k dot is reduced with DPP inside the 16-lane
// row.  With one split the workgroup writes the output; otherwise it writes
// o and (m, l) per head to the caller's score_buf -- the reference's
// scratch argument -- and a second kernel merges the splits.  Nothing is
// allocated.
#include "common.hpp"
#include "head_math.hpp"

#include <cmath>
#include <type_traits>

// Workgroups the split-K grid aims for (splits are also capped by score_buf).
#ifndef FENCE_ATTN_GT_MAX
#define FENCE_ATTN_GT_MAX 2
#endif
#ifndef FENCE_ATTN_TARGET_WG
#define FENCE_ATTN_TARGET_WG 1024
#endif
// 1: fence_gqa_attention_qk_f16_arrive merges in the split launch (one
// launch); 0: it launches the merge kernel as fence_gqa_attention_qk_f16 does
// (an A/B build: `make TAG=noarrive EXTRA=-DFENCE_ATTN_ARRIVE=0`).  Results
// are the same bits either way.
#ifndef FENCE_ATTN_ARRIVE
#define FENCE_ATTN_ARRIVE 1
#endif
// Words between two arrival counters (at most FENCE_ARRIVE_WORDS_PER_HEAD):
// every counter on a cache line of its own, so the device-scope atomics of
// different head groups do not queue behind one another.
#ifndef FENCE_ATTN_ARRIVE_STRIDE
#define FENCE_ATTN_ARRIVE_STRIDE 64
#endif
static_assert(FENCE_ATTN_ARRIVE_STRIDE >= 1 && FENCE_ATTN_ARRIVE_STRIDE <= FENCE_ARRIVE_WORDS_PER_HEAD,
              "arrival counter stride");
// Sub-chunks of K and V rows a split workgroup holds in flight: 2 loads the
// next sub-chunk's rows while the current one is computed (and the first two
// before the prologue); 1 (kept) loads each sub-chunk after the previous one
// is done.  The arithmetic, and so every result, is the same either way.
// Measured on MI355X, Qwen3-4B decode steps (bench.py --decode-only, 64
// tokens, interleaved runs against a `make TAG=kv2
// EXTRA=-DFENCE_ATTN_KV_BUFS=2` build): 1,706-1,707 us per token with 1
// against 1,717-1,721 with 2, whose split kernel needs 161 VGPRs (92).
#ifndef FENCE_ATTN_KV_BUFS
#define FENCE_ATTN_KV_BUFS 1
#endif
static_assert(FENCE_ATTN_KV_BUFS == 1 || FENCE_ATTN_KV_BUFS == 2, "K/V buffers: 1 or 2");

namespace fence {
namespace {

#ifndef FENCE_ATTN_THREADS
#define FENCE_ATTN_THREADS 256
#endif
constexpr int kThreads = FENCE_ATTN_THREADS;  // split kernel workgroup
#ifndef FENCE_ATTN_PPG
#define FENCE_ATTN_PPG 4  // positions per 16-lane group per sub-chunk
#endif

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

// 2^x by the hardware's v_exp_f32.  Scores are kept in log2 units
// (s * scale * log2 e), so exp(s_t - m) is one instruction -- the form the
// reference's fast-math expf also takes (2^(x log2 e)).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Operands of the q and k preparation a split launch does itself when ROPE
// is set (fence_gqa_attention_qk_f16): qk_norm_rope_store_kv's work
// (head_ops.hip) for the token at position pos = seq_len - 1, whose q the
// kernel then reads unprepared.
struct QkIn {
    const float* k;   // [n_kv][128]: the token's k and v, before norm and RoPE
    const float* v;
    const float* wq;  // [128]: QK-norm weights, or both null (RoPE only)
    const float* wk;
    uint16_t* kc;     // the caches, writable: row pos receives the token's k and v
    uint16_t* vc;
    float eps;
    InvFreq tab;
};

// Reduce-scatter over the 16 lanes of a row: N values per lane in (N a power
// of two, at most 16), and every lane leaves with the row's sum of one of
// them, value idx(i) = sum over the halving steps s of bit (3 - s) of lane
// i times N / 2^(s + 1).  Step s pairs lane i with lane i ^ 15, i ^ 7, i ^ 2,
// i ^ 1 (DPP row_mirror, row_half_mirror, quad_perm xor 2, xor 1): the lane
// whose step bit is 0 keeps the lower half of its values and adds its
// partner's lower half, the other the upper halves; once one value is left a
// step just adds the partner's.  All 64 lanes must be active.
template <int S, int M>
__device__ __forceinline__ float row_reduce_scatter(const float* v, int sl) {
    if constexpr (S == 4) {
        static_assert(M == 1, "at most 16 values");
        return v[0];
    } else {
        constexpr int kCtrl = S == 0 ? kDppMirror : S == 1 ? kDppHalfMirror : S == 2 ? kDppQuadXor2 : kDppQuadXor1;
        if constexpr (M == 1) {
            const float w = v[0] + dpp<kCtrl>(v[0]);
            return row_reduce_scatter<S + 1, 1>(&w, sl);
        } else {
            constexpr int H = M / 2;
            const bool upper = (sl >> (3 - S)) & 1;
            float w[H];
#pragma unroll
            for (int k = 0; k < H; ++k) {
                const float keep = upper ? v[k + H] : v[k];
                const float send = upper ? v[k] : v[k + H];
                w[k] = keep + dpp<kCtrl>(send);
            }
            return row_reduce_scatter<S + 1, H>(w, sl);
        }
    }
}

// The index of the value row_reduce_scatter<0, N> leaves in lane sl.
template <int N>
__device__ __forceinline__ int row_scatter_index(int sl) {
    int idx = 0;
#pragma unroll
    for (int s = 0, h = N / 2; h >= 1; ++s, h /= 2) idx += ((sl >> (3 - s)) & 1) * h;
    return idx;
}

// Split partials in ws (16-byte aligned), n_q * splits * (128 + 2) floats:
// the o rows [n_q][splits][128], then the (m, l) pairs [n_q][splits][2].
constexpr int kHD = 128;
__device__ __forceinline__ int64_t partial_o_at(int h, int splits, int split) {
    return (static_cast<int64_t>(h) * splits + split) * kHD;
}
__device__ __forceinline__ int64_t partial_ml_at(int n_q, int h, int splits, int split) {
    return static_cast<int64_t>(n_q) * splits * kHD + (static_cast<int64_t>(h) * splits + split) * 2;
}

// Buffer resource word 3 for raw dword accesses (DATA_FORMAT 32), and the
// cache policy (sc1) of an agent-scope atomic load: the arrival merge reads
// partials that workgroups on other XCDs -- other L2s -- of the same launch
// wrote.  A buffer access past the resource's size reads 0 and never faults.
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kPolicyDevice = 16;

// One wave's merge of one query head's splits (at most kWave) over dims
// [64 half, 64 half + 64).  Lane (sg, j) = (lane / 16, lane % 16) loads dims
// 4j .. 4j + 3 of splits sg, sg + 4, .. (one 128-bit load each, all issued
// before any use) and lane s the (m, l) of split s.  M = max m_s, c_s =
// 2^(m_s - M) (0 for an empty split), L = sum l_s c_s by a DPP reduction; each
// lane adds c_b o_b over its splits in order, the four lane groups are added
// as (sg0 + sg1) + (sg2 + sg3), and every lane returns the four dims' o / L.
// Shared by the merge kernel and the split kernel's last-arrival merge, so
// both give the same bits.
// A wave-uniform pointer as the compiler's uniform value (lane 0's copy), so
// a buffer resource built from it needs no per-lane loop.
__device__ __forceinline__ float* uniform_ptr(const float* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<float*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// o_head and ml_head are wave-uniform.
template <int POLICY>
__device__ __forceinline__ f4 merge_head_half(const float* o_head, const float* ml_head, int splits, int half,
                                              int lane) {
    const __amdgpu_buffer_rsrc_t ro =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(o_head), 0, splits * kHD * 4, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rml =
        __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(ml_head), 0, splits * 8, kRsrcWord3);
    const int j = lane & 15, sg = lane >> 4;
    const f2 ml = __builtin_bit_cast(f2, __builtin_amdgcn_raw_buffer_load_b64(rml, lane * 8, 0, POLICY));
    // Every load is issued and used, with no branch, so the wait counter
    // stays exact and (m, l)'s arithmetic below overlaps the o loads; splits
    // past the last read 0 and weigh 0, adding 0 * 0.
    f4 ov[kWave / 4];
#pragma unroll
    for (int i = 0; i < kWave / 4; ++i) {
        const int at = ((sg + 4 * i) * kHD + 64 * half + 4 * j) * 4;
        ov[i] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(ro, at, 0, POLICY));
    }
    const bool on = lane < splits;
    const float M = wave_reduce(on ? ml.x : -__builtin_inff(), OpMax{});
    const float c = (!on || ml.y == 0.0f) ? 0.0f : exp2_hw(ml.x - M);  // an empty split weighs 0
    const float L = wave_reduce(on ? ml.y * c : 0.0f, OpAdd{});
    // Lane (sg, j) takes c of split sg + 4j; step i then broadcasts lane
    // (sg, i)'s copy over the 16-lane row (DPP row_newbcast): c of split
    // sg + 4i, with no LDS round trip per step.
    const float ct = __shfl(c, sg + 4 * j, kWave);
    f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    static_for<0, kWave / 4>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        const float cb = dpp<kDppRowNewBcast0 + i>(ct);
        acc.x = __builtin_fmaf(cb, ov[i].x, acc.x);
        acc.y = __builtin_fmaf(cb, ov[i].y, acc.y);
        acc.z = __builtin_fmaf(cb, ov[i].z, acc.z);
        acc.w = __builtin_fmaf(cb, ov[i].w, acc.w);
    });
#pragma unroll
    for (int m = 16; m <= 32; m *= 2) {
        acc.x += __shfl_xor(acc.x, m, kWave);
        acc.y += __shfl_xor(acc.y, m, kWave);
        acc.z += __shfl_xor(acc.z, m, kWave);
        acc.w += __shfl_xor(acc.w, m, kWave);
    }
    if (L == 0.0f) return f4{0.0f, 0.0f, 0.0f, 0.0f};
    return f4{acc.x / L, acc.y / L, acc.z / L, acc.w / L};
}

// merge_head_half's outputs: lane (sg, j) writes dim 64 half + 4j + sg.
__device__ __forceinline__ void write_head_half(float* out, uint16_t* out16, int h, int half, int lane, f4 r) {
    const int sg = lane >> 4;
    const float v = sg == 0 ? r.x : sg == 1 ? r.y : sg == 2 ? r.z : r.w;
    const int64_t at = static_cast<int64_t>(h) * kHD + 64 * half + 4 * (lane & 15) + sg;
    if (out) out[at] = v;
    if (out16) out16[at] = f32_to_f16_bits(v);
}

// Split kernel: grid (n_kv * head_groups, splits); HD = 128.  The workgroup
// walks its positions in sub-chunks of kSub (= 64): (A) every 16-lane group
// scores its positions for the GT heads into LDS, (B) every wave takes each
// head's sub-chunk maximum, exponentials and sum (lane t: position t; all
// waves compute the same values) and rescales its running sum, (C) every lane
// accumulates p * v for its 8 dims, p_t read from lane t.  One barrier per
// sub-chunk, after (A): the score buffer alternates between two halves.  The
// V rows of a sub-chunk are loaded together with its K rows, before phase A.
// FINAL: one split, write the output; else write (m, l, o) partials to ws.
// ROPE (kRopeNeox / kRopeInter): a prologue applies QK-norm and RoPE to the
// workgroup's GT q heads with the head kernels' arithmetic (head_math.hpp),
// so q is bit-identical to theirs; the workgroups whose range holds position
// pos also prepare that position's k and v in LDS and attend to it from
// there (the cache row is never read), and the first head group's one writes
// the row to the caches.  The first sub-chunk's K and V loads (the first
// two sub-chunks' with FENCE_ATTN_KV_BUFS 2) are issued before the
// prologue, which runs while they are in flight.
// ARRIVE (with !FINAL, at most kWave splits): no merge launch.  The partials
// are written with device-coherent stores (agent-scope atomic stores, which
// write through the XCD's L2); once they have completed, the workgroup bumps
// arrive[its (kv head, head group)], and the workgroup that brings it to
// `splits` -- the last of that head group's splits -- resets it to 0 and
// merges the group's heads itself, reading every split's partials with
// device-coherent loads, in the merge kernel's arithmetic.  No workgroup ever
// waits for another.
template <int GT, bool FINAL, int ROPE, bool ARRIVE = false>
__global__ __launch_bounds__(kThreads) void attn_split_kernel(float* __restrict__ out, uint16_t* __restrict__ out16,
                                                              float* __restrict__ ws,
                                                              const float* __restrict__ q,
                                                              const uint16_t* __restrict__ kc,
                                                              const uint16_t* __restrict__ vc, int n_q, int n_kv,
                                                              int seq_len, int chunk, float scale2, const QkIn qk,
                                                              uint32_t* __restrict__ arrive) {
    constexpr int HD = 128;
    constexpr int HALF = HD / 2;
    constexpr int G = HD / 8;              // prologue lanes (units) per head
    constexpr int kPG = kThreads / 16;     // position groups (16 lanes each)
    constexpr int kPPG = FENCE_ATTN_PPG;   // positions per group per sub-chunk
    constexpr int kSub = kPG * kPPG;       // positions per sub-chunk
    constexpr bool QK = ROPE != kRopeNone;
    constexpr int kUnits = G * (GT + 1);   // prologue: the GT q heads' units, then the k head's
    static_assert(!QK || (kThreads >= 3 * kWave && kUnits <= 2 * kWave), "prologue lanes");
    static_assert(kSub == kWave, "one position of a sub-chunk per lane in (B)");
    __shared__ float sp[2][GT][kSub];      // scores of even / odd sub-chunks
    __shared__ __align__(16) float xo[kPG][GT][HD];
    __shared__ __align__(16) float qcs[QK ? HD : 1];            // prologue: cos[HALF] then sin[HALF]
    __shared__ __align__(16) float qs[QK ? GT : 1][HD];         // prologue: the prepared q heads
    __shared__ __align__(16) uint16_t kvn[QK ? 2 : 1][HD];      // prologue: position pos's k, v (binary16)
    const int group = n_q / n_kv;
    const int head_groups = (group + GT - 1) / GT;
    // The head_groups workgroups of one (kv head, split) read the same K and V
    // rows.  Workgroups are dispatched to the 8 XCDs round-robin by linear
    // id, and each XCD has its own L2, so with n_kv a multiple of 8 the ids
    // are remapped to put those workgroups 8 ids apart -- on one XCD, where
    // the later reads hit the earlier ones' lines (measured: 12.5 -> 12.0 us
    // at 2916 positions, 14.4 -> 13.7 us at 4096, split + merge).  The work of
    // each workgroup, and so every result, is unchanged.
    int bx = blockIdx.x, by = blockIdx.y;
    if (head_groups > 1 && n_kv % 8 == 0) {
        const int L = blockIdx.x + gridDim.x * blockIdx.y;
        const int r = L >> 3;
        const int P = (r / head_groups) * 8 + (L & 7);  // (kv head, split) = (P % n_kv, P / n_kv)
        bx = (P % n_kv) * head_groups + r % head_groups;
        by = P / n_kv;
    }
    const int kvh = bx / head_groups;
    const int hgi = bx % head_groups;                        // head group within the kv head's
    const int h0 = kvh * group + hgi * GT;                   // first query head of this workgroup
    const int ng = min(GT, kvh * group + group - h0);        // heads present (GT or fewer)
    const int split = by;
    const int t_begin = split * chunk;
    const int t_end = min(seq_len, t_begin + chunk);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int pg = threadIdx.x >> 4;  // position group
    const int sl = lane & 15;         // dims [8 sl, 8 sl + 8)
    const int64_t kv_dim = static_cast<int64_t>(n_kv) * HD;
    const int pos = seq_len - 1;
    const bool has_pos = QK && t_begin <= pos && pos < t_end;  // workgroup-uniform

    float qv[GT][8];
    if constexpr (!QK) {
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            const int h = h0 + (g < ng ? g : 0);  // a missing head repeats head h0 and is not written
            const f4 a = *reinterpret_cast<const f4*>(q + static_cast<int64_t>(h) * HD + 8 * sl);
            const f4 b = *reinterpret_cast<const f4*>(q + static_cast<int64_t>(h) * HD + 8 * sl + 4);
            qv[g][0] = a.x, qv[g][1] = a.y, qv[g][2] = a.z, qv[g][3] = a.w;
            qv[g][4] = b.x, qv[g][5] = b.y, qv[g][6] = b.z, qv[g][7] = b.w;
        }
    }
    float o[GT][8];
#pragma unroll
    for (int g = 0; g < GT; ++g)
#pragma unroll
        for (int i = 0; i < 8; ++i) o[g][i] = 0.0f;
    // running maximum and sum per head: every wave holds the same values
    float hm[GT], hl[GT];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        hm[g] = -__builtin_inff();
        hl[g] = 0.0f;
    }
    int sub = 0;  // sub-chunks processed: sp[sub & 1] is this one's

    const uint16_t* kbase = kc + static_cast<int64_t>(kvh) * HD + 8 * sl;
    const uint16_t* vbase = vc + static_cast<int64_t>(kvh) * HD + 8 * sl;
    constexpr int NB = FENCE_ATTN_KV_BUFS;
    h8 kbuf[NB][kPPG], vbuf[NB][kPPG];
    bool onbuf[NB][kPPG];
    using Slot0 = std::integral_constant<int, 0>;
    using Slot1 = std::integral_constant<int, NB - 1>;
    // The sub-chunk's K and V rows into buffer `slot`, all loads first.
    // Clamped: a valid cached position (row 0 for an empty range); with ROPE
    // never row pos, which this launch is writing, unless pos is 0.
    const int t_fill = (t_begin < t_end && !(QK && t_begin == pos)) ? t_begin : 0;
    auto load_kv = [&](int t0, auto slot) {
        h8(&kr)[kPPG] = kbuf[decltype(slot)::value];
        h8(&vr)[kPPG] = vbuf[decltype(slot)::value];
        bool(&on)[kPPG] = onbuf[decltype(slot)::value];
#pragma unroll
        for (int i = 0; i < kPPG; ++i) {
            const int t = t0 + pg + kPG * i;
            on[i] = t < t_end;
            const int64_t tc = (on[i] && !(QK && t == pos)) ? t : t_fill;
            kr[i] = __builtin_nontemporal_load(reinterpret_cast<const h8*>(kbase + tc * kv_dim));
            vr[i] = __builtin_nontemporal_load(reinterpret_cast<const h8*>(vbase + tc * kv_dim));
        }
    };
    auto process = [&](int t0, auto slot) {
        h8(&kr)[kPPG] = kbuf[decltype(slot)::value];
        h8(&vr)[kPPG] = vbuf[decltype(slot)::value];
        const bool(&on)[kPPG] = onbuf[decltype(slot)::value];
        if constexpr (QK) {
            if (has_pos) {  // position pos from the prologue's rows
#pragma unroll
                for (int i = 0; i < kPPG; ++i) {
                    if (t0 + pg + kPG * i == pos) {
                        kr[i] = *reinterpret_cast<const h8*>(&kvn[0][8 * sl]);
                        vr[i] = *reinterpret_cast<const h8*>(&kvn[1][8 * sl]);
                    }
                }
            }
        }
        // A masked slot's clamped row may be the one this launch is writing
        // (position 0) or hold any bits; its weight is 0, and so is its V.
#pragma unroll
        for (int i = 0; i < kPPG; ++i) vr[i] = on[i] ? vr[i] : h8(0);
        // (A) scores, in log2 units: each lane's 8-dim partial dots of its
        // kPPG positions and GT heads, then one reduce-scatter over the row,
        // after which lane sl holds the score of (position, head) index
        // row_scatter_index(sl) and the first lane of each pair writes it
        float(&spb)[GT][kSub] = sp[sub & 1];
        constexpr int kDots = kPPG * GT;  // index i * GT + g
        static_assert(kDots <= 16 && (kDots & (kDots - 1)) == 0, "scores per row: a power of two, at most 16");
        float dots[kDots];
#pragma unroll
        for (int i = 0; i < kPPG; ++i) {
            float kf[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) kf[k] = static_cast<float>(kr[i][k]);
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                float d = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; ++k) d = __builtin_fmaf(qv[g][k], kf[k], d);
                dots[i * GT + g] = d;
            }
        }
        {
            const float d = row_reduce_scatter<0, kDots>(dots, sl);
            const int idx = row_scatter_index<kDots>(sl);
            const int i = idx / GT, g = idx % GT;
            constexpr int kCopies = 16 / kDots;  // lanes holding each score
            if (sl % kCopies == 0) spb[g][pg + kPG * i] = t0 + pg + kPG * i < t_end ? d * scale2 : -__builtin_inff();
        }
        // One barrier per sub-chunk: the next sub-chunk writes the other
        // buffer, and the one after that comes after the next barrier.
        __syncthreads();
        // (B) every wave, every head: lane t holds position t0 + t -- the
        // sub-chunk's maximum, the weights and their sum, each computed the
        // same way in every wave, so all waves keep the same running values
        float pw[GT], cw[GT], sv[GT], mx[GT], sm[GT];
#pragma unroll
        for (int g = 0; g < GT; ++g) sv[g] = spb[g][lane];
#pragma unroll
        for (int g = 0; g < GT; ++g) mx[g] = wave_reduce(fmaxf(-__builtin_inff(), sv[g]), OpMax{});
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            const float mn = fmaxf(hm[g], mx[g]);
            pw[g] = sv[g] == -__builtin_inff() ? 0.0f : exp2_hw(sv[g] - mn);
            cw[g] = hl[g] == 0.0f ? 0.0f : exp2_hw(hm[g] - mn);  // nothing seen yet: no old weight
            hm[g] = mn;
        }
#pragma unroll
        for (int g = 0; g < GT; ++g) sm[g] = wave_reduce(pw[g], OpAdd{});
#pragma unroll
        for (int g = 0; g < GT; ++g) hl[g] = hl[g] * cw[g] + sm[g];
        // (C) o = o * c + sum_t p_t v_t over the lane's dims.  Lane (row,
        // i) takes p of its row's position i (pg + kPG i, from lane t of (B)),
        // then step i broadcasts it over the row (DPP row_newbcast).
#pragma unroll
        for (int g = 0; g < GT; ++g) {
#pragma unroll
            for (int k = 0; k < 8; ++k) o[g][k] *= cw[g];
        }
        float pq[GT];
#pragma unroll
        for (int g = 0; g < GT; ++g) pq[g] = __shfl(pw[g], pg + kPG * (sl % kPPG), kWave);
        static_for<0, kPPG>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            float vf[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) vf[k] = static_cast<float>(vr[i][k]);
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                const float p = dpp<kDppRowNewBcast0 + i>(pq[g]);
#pragma unroll
                for (int k = 0; k < 8; ++k) o[g][k] = __builtin_fmaf(p, vf[k], o[g][k]);
            }
        });
        ++sub;
    };

    // Unit u < kUnits: q head g = u / G (u < G * GT), else the k head;
    // elements [4i, 4i + 4) and [HALF + 4i, HALF + 4i + 4), i = u % G.
    // Whole waves compute (the DPP rows need every lane); lanes past the
    // units repeat the k unit and store nothing.  Wave 2 computes the pair
    // angles' cos and sin meanwhile.  The prologue's loads are issued before
    // the K and V loads: loads complete in issue order for the wait counter,
    // so the prologue then runs while the K and V rows are still in flight.
    const int u = threadIdx.x;
    const bool unit_wave = QK && wave * kWave < kUnits;  // wave-uniform
    const bool isk = u >= G * GT;
    const int iu = u % G;
    const int gu = isk ? 0 : u / G;
    f4 a, b, va, vb, wa, wb;
    float freq = 0.0f;
    if constexpr (QK) {
        if (unit_wave) {
            const float* src = isk ? qk.k + static_cast<int64_t>(kvh) * HD
                                   : q + static_cast<int64_t>(h0 + (gu < ng ? gu : 0)) * HD;
            const float* vsrc = qk.v + static_cast<int64_t>(kvh) * HD;
            a = ld4<false>(src + 4 * iu);
            b = ld4<false>(src + HALF + 4 * iu);
            va = ld4<false>(vsrc + 4 * iu);
            vb = ld4<false>(vsrc + HALF + 4 * iu);
            if (qk.wq) {  // launch-uniform
                const float* w = isk ? qk.wk : qk.wq;
                wa = ld4<false>(w + 4 * iu);
                wb = ld4<false>(w + HALF + 4 * iu);
            }
        } else if (wave == 2) {
            freq = qk.tab.v[lane];
        }
    }
    // Issued whether or not the range is empty (then clamped and unused), so
    // that every path reaches the prologue's waits with the same loads in
    // flight and they wait for the prologue's own loads only.
    load_kv(t_begin, Slot0{});
    if (NB == 2 && t_begin + kSub < t_end) load_kv(t_begin + kSub, Slot1{});
    if constexpr (QK) {
        const int i = iu, g = gu;
        if (unit_wave) {
            if (qk.wq) head_norm_unit<G>(a, b, wa, wb, qk.eps);
        } else if (wave == 2) {
            float sn, cn;
            sincos_angle(static_cast<float>(pos) * freq, &sn, &cn);
            qcs[lane] = cn;
            qcs[HALF + lane] = sn;
        }
        __syncthreads();  // qcs
        if (unit_wave) {
            rope_unit<ROPE, G>(a, b, qcs, i);
            if (!isk) {
                *reinterpret_cast<f4*>(&qs[g][4 * i]) = a;
                *reinterpret_cast<f4*>(&qs[g][HALF + 4 * i]) = b;
            } else if (u < kUnits && has_pos) {
                st_h4<false>(&kvn[0][4 * i], a);
                st_h4<false>(&kvn[0][HALF + 4 * i], b);
                st_h4<false>(&kvn[1][4 * i], va);
                st_h4<false>(&kvn[1][HALF + 4 * i], vb);
                if (hgi == 0) {  // one writer per kv head
                    const int64_t at = static_cast<int64_t>(pos) * kv_dim + static_cast<int64_t>(kvh) * HD;
                    st_h4<false>(qk.kc + at + 4 * i, a);
                    st_h4<false>(qk.kc + at + HALF + 4 * i, b);
                    st_h4<false>(qk.vc + at + 4 * i, va);
                    st_h4<false>(qk.vc + at + HALF + 4 * i, vb);
                }
            }
        }
        __syncthreads();  // qs, kvn
#pragma unroll
        for (int g = 0; g < GT; ++g) {
            const f4 a = *reinterpret_cast<const f4*>(&qs[g][8 * sl]);
            const f4 b = *reinterpret_cast<const f4*>(&qs[g][8 * sl + 4]);
            qv[g][0] = a.x, qv[g][1] = a.y, qv[g][2] = a.z, qv[g][3] = a.w;
            qv[g][4] = b.x, qv[g][5] = b.y, qv[g][6] = b.z, qv[g][7] = b.w;
        }
    }
    if constexpr (NB == 1) {
        if (t_begin < t_end) process(t_begin, Slot0{});
        for (int t0 = t_begin + kSub; t0 < t_end; t0 += kSub) {
            load_kv(t0, Slot0{});
            process(t0, Slot0{});
        }
    } else {
        // sub-chunks alternate buffers; each buffer is refilled with the
        // sub-chunk after next as soon as it has been computed
        for (int t0 = t_begin; t0 < t_end; t0 += 2 * kSub) {
            process(t0, Slot0{});
            if (t0 + 2 * kSub < t_end) load_kv(t0 + 2 * kSub, Slot0{});
            if (t0 + kSub < t_end) {
                process(t0 + kSub, Slot1{});
                if (t0 + 3 * kSub < t_end) load_kv(t0 + 3 * kSub, Slot1{});
            }
        }
    }

    // Sum the position groups' outputs (they share the running maximum).
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        f4 lo, hi;
        lo.x = o[g][0], lo.y = o[g][1], lo.z = o[g][2], lo.w = o[g][3];
        hi.x = o[g][4], hi.y = o[g][5], hi.z = o[g][6], hi.w = o[g][7];
        *reinterpret_cast<f4*>(&xo[pg][g][8 * sl]) = lo;
        *reinterpret_cast<f4*>(&xo[pg][g][8 * sl + 4]) = hi;
    }
    __syncthreads();
    // thread (g, d): one output element of one head
    for (int e = threadIdx.x; e < GT * HD; e += kThreads) {
        const int g = e / HD, d = e % HD;
        if (g >= ng) continue;
        float acc = 0.0f;
        for (int k = 0; k < kPG; ++k) acc += xo[k][g][d];
        float l = hl[0], mg = hm[0];
#pragma unroll
        for (int k = 1; k < GT; ++k) {
            l = g == k ? hl[k] : l;
            mg = g == k ? hm[k] : mg;
        }
        const int h = h0 + g;
        if constexpr (FINAL) {
            const float r = l == 0.0f ? 0.0f : acc / l;
            if (out) out[static_cast<int64_t>(h) * HD + d] = r;
            if (out16) out16[static_cast<int64_t>(h) * HD + d] = f32_to_f16_bits(r);
        } else {
            // partial of (head h, split): o[HD], then (m, l)
            const int splits = static_cast<int>(gridDim.y);
            float* po = ws + partial_o_at(h, splits, split);
            float* pml = ws + partial_ml_at(n_q, h, splits, split);
            if constexpr (ARRIVE) {
                if (d == 0) {
                    __hip_atomic_store(pml, mg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(pml + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                __hip_atomic_store(po + d, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                if (d == 0) {
                    pml[0] = mg;
                    pml[1] = l;
                }
                po[d] = acc;
            }
        }
    }
    if constexpr (!FINAL && ARRIVE) {
        __shared__ uint32_t last;
        // Every wave's partial stores have completed (gfx9 counts stores in
        // vmcnt) before the one arrival below is made.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0) {
            const uint32_t before = __hip_atomic_fetch_add(arrive + bx * FENCE_ATTN_ARRIVE_STRIDE, 1u, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
            last = before + 1 == gridDim.y ? 1u : 0u;
        }
        __syncthreads();
        if (last == 0) return;  // workgroup-uniform
        if (threadIdx.x == 0)
            __hip_atomic_store(arrive + bx * FENCE_ATTN_ARRIVE_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // The merge of heads h0 .. h0 + ng - 1: wave w takes head-halves
        // e = w, w + 4, ..: head e / 2, dims [64 (e % 2), 64 (e % 2) + 64).
        const int splits = static_cast<int>(gridDim.y);
        for (int e = wave; e < 2 * ng; e += kThreads / kWave) {
            const int h = h0 + e / 2;
            const f4 r = merge_head_half<kPolicyDevice>(ws + partial_o_at(h, splits, 0),
                                                        ws + partial_ml_at(n_q, h, splits, 0), splits, e % 2, lane);
            write_head_half(out, out16, h, e % 2, lane, r);
        }
    }
}

// Merge kernel: one workgroup of HD threads per query head.  Up to kWave
// splits, wave w merges dims [64 w, 64 w + 64) with merge_head_half.  More
// splits (up to kMaxMergeSplits) take the LDS form, thread d owning dim d:
// (m, l) through LDS, then the o sums eight loads at a time.
constexpr int kMaxMergeSplits = 1024;

__global__ __launch_bounds__(128) void attn_merge_kernel(float* __restrict__ out, uint16_t* __restrict__ out16,
                                                         const float* __restrict__ ws, int n_q, int splits) {
    constexpr int HD = kHD;
    const int h = blockIdx.x, d = threadIdx.x, lane = threadIdx.x & (kWave - 1);
    const float* po = ws + partial_o_at(h, splits, 0);
    const float* pml = ws + partial_ml_at(n_q, h, splits, 0);
    if (splits <= kWave) {
        const int half = threadIdx.x / kWave;
        write_head_half(out, out16, h, half, lane, merge_head_half<0>(po, pml, splits, half, lane));
        return;
    }
    __shared__ float cw[kMaxMergeSplits];
    __shared__ float red[2];
    float m = -__builtin_inff();
    for (int s = d; s < splits; s += HD) m = fmaxf(m, pml[2 * s]);
    m = block_reduce<2>(m, OpMax{}, red);
    __syncthreads();
    float l = 0.0f;
    for (int s = d; s < splits; s += HD) {
        const float ls = pml[2 * s + 1];
        const float c = ls == 0.0f ? 0.0f : exp2_hw(pml[2 * s] - m);
        cw[s] = c;
        l += ls * c;
    }
    l = block_reduce<2>(l, OpAdd{}, red);  // its barrier also publishes cw[]
    float o = 0.0f;
    constexpr int kBatch = 8;
    for (int s0 = 0; s0 < splits; s0 += kBatch) {
        float v[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) v[b] = po[static_cast<int64_t>(s0 + b < splits ? s0 + b : s0) * HD + d];
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
            if (s0 + b < splits) o = __builtin_fmaf(cw[s0 + b], v[b], o);
    }
    const float r = l == 0.0f ? 0.0f : o / l;
    if (out) out[static_cast<int64_t>(h) * HD + d] = r;
    if (out16) out16[static_cast<int64_t>(h) * HD + d] = f32_to_f16_bits(r);
}

// Any head_dim / alignment: one workgroup per query head, the reference's
// three passes with the scores kept in ws (n_q x max_ctx, as the reference).
__global__ __launch_bounds__(256) void attn_generic_kernel(float* __restrict__ out, uint16_t* __restrict__ out16,
                                                           float* __restrict__ ws,
                                                           const float* __restrict__ q,
                                                           const uint16_t* __restrict__ kc,
                                                           const uint16_t* __restrict__ vc, int hd, int n_q,
                                                           int n_kv, int seq_len, int max_ctx, float scale) {
    __shared__ float red[4];
    const int h = blockIdx.x;
    const int kvh = h / (n_q / n_kv);
    const int64_t kv_dim = static_cast<int64_t>(n_kv) * hd;
    float* s = ws + static_cast<int64_t>(h) * max_ctx;
    const float* qh = q + static_cast<int64_t>(h) * hd;
    for (int t = threadIdx.x; t < seq_len; t += 256) {
        const uint16_t* k = kc + t * kv_dim + static_cast<int64_t>(kvh) * hd;
        float dot = 0.0f;
        for (int d = 0; d < hd; ++d) dot = __builtin_fmaf(qh[d], static_cast<float>(__builtin_bit_cast(_Float16, k[d])), dot);
        s[t] = dot * scale;
    }
    float mx = -1e30f;
    for (int t = threadIdx.x; t < seq_len; t += 256) mx = fmaxf(mx, s[t]);
    mx = block_reduce<4>(mx, OpMax{}, red);
    __syncthreads();
    float sum = 0.0f;
    for (int t = threadIdx.x; t < seq_len; t += 256) {
        const float e = expf(s[t] - mx);
        s[t] = e;
        sum += e;
    }
    sum = block_reduce<4>(sum, OpAdd{}, red);
    const float inv = 1.0f / sum;
    __syncthreads();  // every s[t] written above is visible below
    for (int d = threadIdx.x; d < hd; d += 256) {
        float acc = 0.0f;
        for (int t = 0; t < seq_len; ++t)
            acc = __builtin_fmaf(s[t] * inv,
                                 static_cast<float>(__builtin_bit_cast(
                                     _Float16, vc[t * kv_dim + static_cast<int64_t>(kvh) * hd + d])),
                                 acc);
        const float r = seq_len > 0 ? acc : 0.0f;
        if (out) out[static_cast<int64_t>(h) * hd + d] = r;
        if (out16) out16[static_cast<int64_t>(h) * hd + d] = f32_to_f16_bits(r);
    }
}

__global__ __launch_bounds__(256) void store_kv_kernel(uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                       const float* __restrict__ k, const float* __restrict__ v,
                                                       int64_t row, int kv_dim, int vec) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (vec) {
        if (4 * i >= kv_dim) return;
        st_h4<false>(kc + row + 4 * i, *reinterpret_cast<const f4*>(k + 4 * i));
        st_h4<false>(vc + row + 4 * i, *reinterpret_cast<const f4*>(v + 4 * i));
    } else if (i < kv_dim) {
        kc[row + i] = f32_to_f16_bits(k[i]);
        vc[row + i] = f32_to_f16_bits(v[i]);
    }
}

template <int GT, int ROPE>
int launch_split(float* out, uint16_t* out16, float* ws, const float* q, const uint16_t* kc, const uint16_t* vc, int n_q, int n_kv,
                 int seq_len, int64_t ws_floats, float scale, const QkIn& qk, uint32_t* arrive, hipStream_t s) {
    constexpr int HD = 128;
    const int group = n_q / n_kv;
    const int head_groups = (group + GT - 1) / GT;
    const int base_wg = n_kv * head_groups;
    // The partials start at ws's first 16-byte boundary (128-bit merge loads).
    if (ws) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(ws);
        const uintptr_t up = (a + 15) & ~static_cast<uintptr_t>(15);
        ws_floats -= static_cast<int64_t>((up - a) / sizeof(float));
        ws = reinterpret_cast<float*>(up);
    }
    // splits: enough workgroups to fill the GPU, at least one sub-chunk of
    // positions each, and no more partials than score_buf holds
    constexpr int kSubPositions = (kThreads / 16) * FENCE_ATTN_PPG;
    int64_t splits = (FENCE_ATTN_TARGET_WG + base_wg - 1) / base_wg;
    const int64_t by_len = (seq_len + kSubPositions - 1) / kSubPositions;
    if (splits > by_len) splits = by_len;
    const int64_t by_ws = ws ? ws_floats / (static_cast<int64_t>(n_q) * (HD + 2)) : 1;
    if (splits > by_ws) splits = by_ws;
    if (splits < 1) splits = 1;
    if (splits > kMaxMergeSplits) splits = kMaxMergeSplits;
    const int chunk = static_cast<int>((seq_len + splits - 1) / splits);
    const dim3 grid(static_cast<unsigned>(base_wg), static_cast<unsigned>(splits));
    uint32_t* const no_arrive = nullptr;
    if (splits == 1)
        return launch(attn_split_kernel<GT, true, ROPE>, grid, dim3(kThreads), 0, s, out, out16, ws, q, kc, vc, n_q,
                      n_kv, seq_len, chunk, scale, qk, no_arrive);
    if (FENCE_ATTN_ARRIVE && arrive && splits <= kWave)  // the last arrival of each head group merges it
        return launch(attn_split_kernel<GT, false, ROPE, true>, grid, dim3(kThreads), 0, s, out, out16, ws, q, kc,
                      vc, n_q, n_kv, seq_len, chunk, scale, qk, arrive);
    if (int st = launch(attn_split_kernel<GT, false, ROPE>, grid, dim3(kThreads), 0, s, out, out16, ws, q, kc, vc,
                        n_q, n_kv, seq_len, chunk, scale, qk, no_arrive))
        return st;
    return launch(attn_merge_kernel, dim3(static_cast<unsigned>(n_q)), dim3(HD), 0, s, out, out16, ws, n_q,
                  static_cast<int>(splits));
}

// The split launch for GT heads per workgroup, with the q/k prologue of
// style `rope` when qk is set.
template <int GT>
int launch_split_qk(float* out, uint16_t* out16, float* ws, const float* q, const uint16_t* kc, const uint16_t* vc,
                    int n_q, int n_kv, int seq_len, int64_t ws_floats, float scale, const QkIn* qk, int rope,
                    uint32_t* arrive, hipStream_t s) {
    if (!qk)
        return launch_split<GT, kRopeNone>(out, out16, ws, q, kc, vc, n_q, n_kv, seq_len, ws_floats, scale, QkIn{},
                                           arrive, s);
    if (rope == kRopeNeox)
        return launch_split<GT, kRopeNeox>(out, out16, ws, q, kc, vc, n_q, n_kv, seq_len, ws_floats, scale, *qk,
                                           arrive, s);
    return launch_split<GT, kRopeInter>(out, out16, ws, q, kc, vc, n_q, n_kv, seq_len, ws_floats, scale, *qk, arrive,
                                        s);
}

}  // namespace

// out (fp32) and/or out16 (its binary16 rounding, the f32_to_f16 of
// src/model/qwen3.cu:310 fused) receive the result.
// ws holds ws_floats floats (the reference's score_buf: n_q * max_ctx).
// qk (with style rope): q is unprepared and the launch applies QK-norm, RoPE
// and the KV store of position seq_len - 1 itself; only on the vector path
// (the caller checks vec_attention).  arrive (n_q * FENCE_ARRIVE_WORDS_PER_HEAD
// zeroed words, left zeroed): a split launch of at most 64 splits merges them
// itself.
int gqa_attention_launch(float* out, uint16_t* out16, const float* q, const void* kcv, const void* vcv, int hd,
                         int n_q, int n_kv, int seq_len, int max_ctx, float* ws, int64_t ws_floats, hipStream_t s,
                         const QkIn* qk = nullptr, int rope = kRopeNone, uint32_t* arrive = nullptr) {
    if ((!out && !out16) || !q || !kcv || !vcv || hd <= 0 || n_q <= 0 || n_kv <= 0 || (n_q % n_kv) != 0)
        return FENCE_ERROR_INVALID_VALUE;
    if (out16 && !aligned(out16, 2)) return FENCE_ERROR_INVALID_VALUE;
    if (seq_len < 0 || max_ctx < 1 || seq_len > max_ctx) return FENCE_ERROR_INVALID_VALUE;
    const uint16_t* kc = static_cast<const uint16_t*>(kcv);
    const uint16_t* vc = static_cast<const uint16_t*>(vcv);
    if ((out && !aligned(out, 4)) || !aligned(q, 4) || !aligned(kc, 2) || !aligned(vc, 2) || (ws && !aligned(ws, 4)))
        return FENCE_ERROR_INVALID_VALUE;
    const float scale = 1.0f / sqrtf(static_cast<float>(hd));
    const float scale2 = scale * 1.44269504088896340736f;  // scores in log2 units for exp2
    const int group = n_q / n_kv;
    const bool vec = hd == 128 && aligned(q, 16) && aligned(kc, 16) && aligned(vc, 16);
    if (qk && !vec) return FENCE_ERROR_INVALID_VALUE;
    if (vec) {
        if (FENCE_ATTN_GT_MAX == 1)
            return launch_split_qk<1>(out, out16, ws, q, kc, vc, n_q, n_kv, seq_len, ws_floats, scale2, qk,
                                      rope, arrive, s);
        if (FENCE_ATTN_GT_MAX == 2 && group >= 2)
            return launch_split_qk<2>(out, out16, ws, q, kc, vc, n_q, n_kv, seq_len, ws_floats, scale2, qk,
                                      rope, arrive, s);
        if (group >= 4)
            return launch_split_qk<4>(out, out16, ws, q, kc, vc, n_q, n_kv, seq_len, ws_floats, scale2, qk,
                                      rope, arrive, s);
        if (group == 2)
            return launch_split_qk<2>(out, out16, ws, q, kc, vc, n_q, n_kv, seq_len, ws_floats, scale2, qk,
                                      rope, arrive, s);
        if (group == 1)
            return launch_split_qk<1>(out, out16, ws, q, kc, vc, n_q, n_kv, seq_len, ws_floats, scale2, qk,
                                      rope, arrive, s);
        // group 3: masked
        return launch_split_qk<4>(out, out16, ws, q, kc, vc, n_q, n_kv, seq_len, ws_floats, scale2, qk,
                                  rope, arrive, s);
    }
    // the generic path keeps scores in score_buf, n_q rows of max_ctx
    if (!ws || ws_floats < static_cast<int64_t>(n_q) * max_ctx) return FENCE_ERROR_INVALID_VALUE;
    return launch(attn_generic_kernel, dim3(static_cast<unsigned>(n_q)), dim3(256), 0, s, out, out16, ws, q, kc, vc,
                  hd, n_q, n_kv, seq_len, max_ctx, scale);
}

int store_kv_launch(void* kcv, void* vcv, const float* k, const float* v, int pos, int kv_dim, int max_ctx,
                    hipStream_t s) {
    if (!kcv || !vcv || !k || !v || kv_dim < 0 || max_ctx < 1 || pos < 0 || pos >= max_ctx)
        return FENCE_ERROR_INVALID_VALUE;
    uint16_t* kc = static_cast<uint16_t*>(kcv);
    uint16_t* vc = static_cast<uint16_t*>(vcv);
    if (!aligned(kc, 2) || !aligned(vc, 2) || !aligned(k, 4) || !aligned(v, 4)) return FENCE_ERROR_INVALID_VALUE;
    if (kv_dim == 0) return FENCE_SUCCESS;
    const int64_t row = static_cast<int64_t>(pos) * kv_dim;
    const int vec = (kv_dim % 4 == 0) && aligned(kc + row, 8) && aligned(vc + row, 8) && aligned(k, 16) &&
                    aligned(v, 16);
    const int items = vec ? kv_dim / 4 : kv_dim;
    return launch(store_kv_kernel, dim3(grid_1d(items, 256)), dim3(256), 0, s, kc, vc, k, v, row, kv_dim, vec);
}

}  // namespace fence

extern "C" int fence_gqa_attention(float* attn_out, const float* q, const void* k_cache, const void* v_cache,
                                   int head_dim, int n_q_heads, int n_kv_heads, int seq_len, int max_ctx,
                                   float* score_buf, hipStream_t stream) {
    if (!attn_out) return FENCE_ERROR_INVALID_VALUE;
    return fence::gqa_attention_launch(attn_out, nullptr, q, k_cache, v_cache, head_dim, n_q_heads, n_kv_heads,
                                       seq_len, max_ctx, score_buf, static_cast<int64_t>(n_q_heads) * max_ctx,
                                       stream);
}

extern "C" int fence_gqa_attention_f16(float* attn_out, void* out_f16, const float* q, const void* k_cache,
                                       const void* v_cache, int head_dim, int n_q_heads, int n_kv_heads, int seq_len,
                                       int max_ctx, float* score_buf, int64_t score_buf_floats, hipStream_t stream) {
    if (!out_f16 || score_buf_floats < 0) return FENCE_ERROR_INVALID_VALUE;
    if (score_buf_floats == 0) score_buf_floats = static_cast<int64_t>(n_q_heads) * max_ctx;
    return fence::gqa_attention_launch(attn_out, static_cast<uint16_t*>(out_f16), q, k_cache, v_cache, head_dim,
                                       n_q_heads, n_kv_heads, seq_len, max_ctx, score_buf, score_buf_floats, stream);
}

namespace {

// fence_gqa_attention_qk_f16, and with arrive its one-launch form.
int attention_qk_f16(float* attn_out, void* out_f16, float* q, float* k, const float* v, const float* q_norm_w,
                     const float* k_norm_w, void* k_cache, void* v_cache, int head_dim, int n_q_heads, int n_kv_heads,
                     int pos, int max_ctx, float eps, float freq_base, int style, float* score_buf,
                     int64_t score_buf_floats, uint32_t* arrive, hipStream_t stream) {
    using namespace fence;
    if (!out_f16 || !q || !k || !v || !k_cache || !v_cache || score_buf_floats < 0) return FENCE_ERROR_INVALID_VALUE;
    if (pos < 0 || max_ctx < 1 || pos >= max_ctx || n_q_heads <= 0 || n_kv_heads <= 0) return FENCE_ERROR_INVALID_VALUE;
    if ((q_norm_w == nullptr) != (k_norm_w == nullptr)) return FENCE_ERROR_INVALID_VALUE;
    if (style != kRopeNeox && style != kRopeInter) return FENCE_ERROR_INVALID_VALUE;
    if (score_buf_floats == 0) score_buf_floats = static_cast<int64_t>(n_q_heads) * max_ctx;
    uint16_t* o16 = static_cast<uint16_t*>(out_f16);
    // Everything either call would reject is rejected here, before any work:
    // an error never leaves q, k or the caches half updated.
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 2 * kMaxHalf || n_q_heads % n_kv_heads != 0 ||
        !(freq_base > 0.0f) || !std::isfinite(freq_base))
        return FENCE_ERROR_INVALID_VALUE;
    if (!aligned(q, 4) || !aligned(k, 4) || !aligned(v, 4) || !aligned(k_cache, 2) || !aligned(v_cache, 2) ||
        (q_norm_w && (!aligned(q_norm_w, 4) || !aligned(k_norm_w, 4))) || (attn_out && !aligned(attn_out, 4)) ||
        !aligned(o16, 2) || (score_buf && !aligned(score_buf, 4)))
        return FENCE_ERROR_INVALID_VALUE;
    const bool vec_attention = head_dim == 128 && aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16);
    if (!vec_attention && (!score_buf || score_buf_floats < static_cast<int64_t>(n_q_heads) * max_ctx))
        return FENCE_ERROR_INVALID_VALUE;  // the generic kernel keeps every score in score_buf
    const bool fused = vec_attention && aligned(k, 16) && aligned(v, 16) &&
                       (!q_norm_w || (aligned(q_norm_w, 16) && aligned(k_norm_w, 16)));
    if (!fused) {  // the two calls it stands for
        if (int st = fence_qk_norm_rope_store_kv(q, k, v, q_norm_w, k_norm_w, k_cache, v_cache, max_ctx, 1, n_q_heads,
                                                 n_kv_heads, head_dim, eps, nullptr, pos, freq_base, style, stream))
            return st;
        return gqa_attention_launch(attn_out, o16, q, k_cache, v_cache, head_dim, n_q_heads, n_kv_heads, pos + 1,
                                    max_ctx, score_buf, score_buf_floats, stream);
    }
    QkIn qk{};
    qk.k = k;
    qk.v = v;
    qk.wq = q_norm_w;
    qk.wk = k_norm_w;
    qk.kc = static_cast<uint16_t*>(k_cache);
    qk.vc = static_cast<uint16_t*>(v_cache);
    qk.eps = eps;
    rope_inv_freq_host(qk.tab.v, head_dim, freq_base);
    return gqa_attention_launch(attn_out, o16, q, k_cache, v_cache, head_dim, n_q_heads, n_kv_heads, pos + 1, max_ctx,
                                score_buf, score_buf_floats, stream, &qk, style, arrive);
}

}  // namespace

extern "C" int fence_gqa_attention_qk_f16(float* attn_out, void* out_f16, float* q, float* k, const float* v,
                                          const float* q_norm_w, const float* k_norm_w, void* k_cache, void* v_cache,
                                          int head_dim, int n_q_heads, int n_kv_heads, int pos, int max_ctx, float eps,
                                          float freq_base, int style, float* score_buf, int64_t score_buf_floats,
                                          hipStream_t stream) {
    return attention_qk_f16(attn_out, out_f16, q, k, v, q_norm_w, k_norm_w, k_cache, v_cache, head_dim, n_q_heads,
                            n_kv_heads, pos, max_ctx, eps, freq_base, style, score_buf, score_buf_floats, nullptr,
                            stream);
}

extern "C" int fence_gqa_attention_qk_f16_arrive(float* attn_out, void* out_f16, float* q, float* k, const float* v,
                                                 const float* q_norm_w, const float* k_norm_w, void* k_cache,
                                                 void* v_cache, int head_dim, int n_q_heads, int n_kv_heads, int pos,
                                                 int max_ctx, float eps, float freq_base, int style, float* score_buf,
                                                 int64_t score_buf_floats, uint32_t* arrive, hipStream_t stream) {
    if (!arrive || !fence::aligned(arrive, 4)) return FENCE_ERROR_INVALID_VALUE;
    return attention_qk_f16(attn_out, out_f16, q, k, v, q_norm_w, k_norm_w, k_cache, v_cache, head_dim, n_q_heads,
                            n_kv_heads, pos, max_ctx, eps, freq_base, style, score_buf, score_buf_floats, arrive,
                            stream);
}

extern "C" int fence_store_kv(void* k_cache, void* v_cache, const float* k, const float* v, int pos, int kv_dim,
                              int max_ctx, hipStream_t stream) {
    return fence::store_kv_launch(k_cache, v_cache, k, v, pos, kv_dim, max_ctx, stream);
}
