// head_ops.hip -- per-head RMSNorm, RoPE (NeoX and interleaved) and their
// fusions with RMSNorm, on gfx950.
//
// Reference math:
//   per-head norm  rms_norm_per_head, src/kernels/ops.cuh:66-103
//   RoPE NeoX      apply_rope,        src/kernels/ops.cuh:115-177
//   RoPE interleaved: pairs (2p, 2p+1) of the comment, src/kernels/ops.cuh:109-113
//   freq[p] = 1.0f / powf(base, (float)(2p)/(float)hd)    (ops.cuh:133),
//   a = (float)pos * freq[p];  x0' = x0 cos a - x1 sin a;  x1' = x0 sin a + x1 cos a.
//
// Two vector kernels.  The streaming kernel (head_dim 128, no row norm, no
// KV store) gives each lane one float4 and each one-wave workgroup two heads
// of a token.  The unit kernel covers the rest, one workgroup (up to 16
// waves) per token: a token's q and k heads are cut into "units" of 8
// floats, elements [4i, 4i+4) and
// [hd/2 + 4i, hd/2 + 4i + 4) of one head (i < hd/8), so a lane holds four
// whole NeoX pairs -- or four whole interleaved pairs -- and never needs a
// partner lane.  A head is hd/8 consecutive lanes, so the per-head sum of
// squares is a DPP reduction inside a 16-lane row (hd = 128).
// freq[] is computed on the host (exactly the reference expression) and
// passed in the kernel arguments; cos/sin of the token's hd/2 angles are
// computed once per token into LDS and shared by all heads, while the
// token's loads are in flight.  The per-head arithmetic is head_math.hpp's,
// which attention.hip shares.
#include "common.hpp"
#include "head_math.hpp"

#include <cmath>

#ifndef FENCE_HEAD_SLOTS
#define FENCE_HEAD_SLOTS 2
#endif

namespace fence {

enum { kNormNone = 0, kNormRow = 1, kNormHead = 2 };

// Operands of a head-structured op.  qo/qi: q output/input
// [tokens][nq][hd]; k: [tokens][nkv][hd], in place; wq/wk: norm weights.
// With kc set (KV store): the rotated k and the matching v [tokens][nkv][hd]
// are also written as binary16 rows of the caches kc/vc [max_ctx][nkv*hd],
// at the token's position (store_kv, src/kernels/ops.cuh:419-443); a
// position outside [0, max_ctx) stores nothing.
struct HeadArgs {
    float* qo;
    const float* qi;
    float* k;
    const float* wq;
    const float* wk;
    int64_t tokens;
    int nq, nkv;
    float eps;
    const int32_t* positions;
    int pos0;
    uint16_t* kc;
    uint16_t* vc;
    const float* v;
    int max_ctx;
};

namespace {

// MAXS units per lane (exactly: the dispatcher launches MAXS == slots).
template <int ROPE, int NORM, int G, int MAXS, bool KV>
__global__ __launch_bounds__(1024) void head_ops_vec_kernel(const HeadArgs args, InvFreq tab) {
    float* qo = args.qo;
    const float* qi = args.qi;
    float* k = args.k;
    const float* wq = args.wq;
    const float* wk = args.wk;
    const int64_t tokens = args.tokens;
    const int nq = args.nq, nkv = args.nkv;
    const float eps = args.eps;
    const int32_t* __restrict__ positions = args.positions;
    const int pos0 = args.pos0;
    constexpr int HD = 8 * G;
    constexpr int HALF = 4 * G;
    __shared__ __align__(16) float cs[2 * HALF];  // cos[HALF] then sin[HALF]
    __shared__ float red[16];
    const int T = blockDim.x;
    const int U = (nq + nkv) * G;

    // A lane's slots map to the same (head, unit) in every token, so the
    // norm weights are loaded once per workgroup, before the token loop.
    f4 wa[MAXS], wb[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; ++s) {
        const int u = threadIdx.x + s * T;
        wa[s] = wb[s] = f4(0.0f);
        if (NORM != kNormNone && u < U) {
            const int h = u / G;
            const int i = u % G;
            const bool isq = h < nq;
            if constexpr (NORM == kNormRow) {
                if (isq) {
                    wa[s] = ld4<false>(wq + h * HD + 4 * i);
                    wb[s] = ld4<false>(wq + h * HD + HALF + 4 * i);
                }
            } else if constexpr (NORM == kNormHead) {
                const float* wr = isq ? wq : wk;
                wa[s] = ld4<false>(wr + 4 * i);
                wb[s] = ld4<false>(wr + HALF + 4 * i);
            }
        }
    }

    // the lane's pair frequencies (p = lane, lane + T < hd/2), read out of
    // the kernel arguments once: a lookup issued after the data loads would
    // make the angle wait for all of them (vmcnt drains in order)
    float invf[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int p = threadIdx.x + j * T;
        invf[j] = (ROPE != kRopeNone && p < HALF) ? tab.v[p] : 0.0f;
    }

    for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
        const int pos = positions ? positions[t] : pos0 + static_cast<int>(t);
        const float* qrow_in = qi + t * nq * HD;
        float* qrow_out = qo + t * nq * HD;
        float* krow = k + t * nkv * HD;

        // Every load of the lane is issued before any is consumed, and without
        // branches (a lane past the last unit reloads the last unit and drops
        // the values), so the compiler can count them and start the angles
        // while they are in flight.
        f4 a[MAXS], b[MAXS];
        f4 va_v[KV ? MAXS : 1], vb_v[KV ? MAXS : 1];  // v of the lane's k units (KV store)
#pragma unroll
        for (int s = 0; s < MAXS; ++s) {
            int u = threadIdx.x + s * T;
            u = u < U ? u : U - 1;
            const int h = u / G;
            const int i = u % G;
            const float* src = (h < nq) ? qrow_in + h * HD : krow + (h - nq) * HD;
            a[s] = ld4<true>(src + 4 * i);
            b[s] = ld4<true>(src + HALF + 4 * i);
            if constexpr (KV) {  // a q unit reads head 0's v and drops it
                const float* vsrc = args.v + t * nkv * HD + (h < nq ? 0 : (h - nq) * HD);
                va_v[s] = ld4<true>(vsrc + 4 * i);
                vb_v[s] = ld4<true>(vsrc + HALF + 4 * i);
            }
        }

        if constexpr (ROPE != kRopeNone) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int p = threadIdx.x + j * T;
                if (p < HALF) {
                    float sn, cn;
                    sincos_angle(static_cast<float>(pos) * invf[j], &sn, &cn);
                    cs[p] = cn;
                    cs[HALF + p] = sn;
                }
            }
        }

        float rrow = 1.0f;
        if constexpr (NORM == kNormRow) {
            float ss = 0.0f;
#pragma unroll
            for (int s = 0; s < MAXS; ++s) {
                const int u = threadIdx.x + s * T;
                if (u < nq * G) ss += dot4(a[s]) + dot4(b[s]);
            }
            const float tot = block_reduce_dyn(ss, OpAdd(), red);
            rrow = rsqrtf(tot / static_cast<float>(nq * HD) + eps);
        }

        float rh[MAXS];
        if constexpr (NORM == kNormHead) {
#pragma unroll
            for (int s = 0; s < MAXS; ++s) {
                const float tot = group_reduce<G>(dot4(a[s]) + dot4(b[s]), OpAdd());
                rh[s] = head_rscale(tot, static_cast<float>(HD), eps);
            }
        }

        if constexpr (ROPE != kRopeNone || NORM == kNormRow) __syncthreads();

#pragma unroll
        for (int s = 0; s < MAXS; ++s) {
            const int u = threadIdx.x + s * T;
            if (u >= U) continue;
            const int h = u / G;
            const int i = u % G;
            const bool isq = h < nq;
            f4 va = a[s];
            f4 vb = b[s];
            if constexpr (NORM == kNormRow) {
                if (isq) {
                    va = (wa[s] * va) * rrow;
                    vb = (wb[s] * vb) * rrow;
                }
            } else if constexpr (NORM == kNormHead) {
                va = (wa[s] * va) * rh[s];
                vb = (wb[s] * vb) * rh[s];
            }
            rope_unit<ROPE, G>(va, vb, cs, i);
            float* dst = isq ? qrow_out + h * HD : krow + (h - nq) * HD;
            st4<true>(dst + 4 * i, va);
            st4<true>(dst + HALF + 4 * i, vb);
            if constexpr (KV) {
                if (!isq && pos >= 0 && pos < args.max_ctx) {
                    const int64_t at = static_cast<int64_t>(pos) * nkv * HD + (h - nq) * HD;
                    st_h4<false>(args.kc + at + 4 * i, va);
                    st_h4<false>(args.kc + at + HALF + 4 * i, vb);
                    st_h4<false>(args.vc + at + 4 * i, va_v[s]);
                    st_h4<false>(args.vc + at + HALF + 4 * i, vb_v[s]);
                }
            }
        }
        __syncthreads();  // cs[] and red[] are rewritten for the next token
    }
}

// Any head_dim and alignment.  One workgroup per token, one wave per head.
template <int ROPE, int NORM>
__global__ __launch_bounds__(256) void head_ops_scalar_kernel(const HeadArgs args, int hd, InvFreq tab) {
    float* qo = args.qo;
    const float* qi = args.qi;
    float* k = args.k;
    const float* wq = args.wq;
    const float* wk = args.wk;
    const int64_t tokens = args.tokens;
    const int nq = args.nq, nkv = args.nkv;
    const float eps = args.eps;
    const int32_t* positions = args.positions;
    const int pos0 = args.pos0;
    __shared__ float red[4];
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int half = hd / 2;
    for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
        const int pos = positions ? positions[t] : pos0 + static_cast<int>(t);
        const float* qrow_in = qi + t * nq * hd;
        float* qrow_out = qo + t * nq * hd;
        float* krow = k + t * nkv * hd;

        float rrow = 1.0f;
        if constexpr (NORM == kNormRow) {
            float ss = 0.0f;
            for (int e = threadIdx.x; e < nq * hd; e += 256) ss += qrow_in[e] * qrow_in[e];
            const float tot = block_reduce<4>(ss, OpAdd(), red);
            rrow = rsqrtf(tot / static_cast<float>(nq * hd) + eps);
        }

        for (int h = wave; h < nq + nkv; h += 4) {
            const bool isq = h < nq;
            const float* src = isq ? qrow_in + h * hd : krow + (h - nq) * hd;
            float* dst = isq ? qrow_out + h * hd : krow + (h - nq) * hd;
            const float* wr = nullptr;
            float r = 1.0f;
            if constexpr (NORM == kNormRow) {
                if (isq) {
                    wr = wq + h * hd;
                    r = rrow;
                }
            } else if constexpr (NORM == kNormHead) {
                wr = isq ? wq : wk;
                float ss = 0.0f;
                for (int e = lane; e < hd; e += kWave) ss += src[e] * src[e];
                r = head_rscale(wave_reduce(ss, OpAdd()), static_cast<float>(hd), eps);
            }
            // KV store of this k head: the row of the token's position
            const bool kv = args.kc && !isq && pos >= 0 && pos < args.max_ctx;
            const int64_t at = static_cast<int64_t>(pos) * nkv * hd + (h - nq) * hd;
            if (kv) {
                const float* vsrc = args.v + t * nkv * hd + (h - nq) * hd;
                for (int e = lane; e < hd; e += kWave) args.vc[at + e] = f32_to_f16_bits(vsrc[e]);
            }
            if constexpr (ROPE == kRopeNone) {
                for (int e = lane; e < hd; e += kWave) {
                    const float val = wr ? (wr[e] * src[e]) * r : src[e];
                    dst[e] = val;
                    if (kv) args.kc[at + e] = f32_to_f16_bits(val);
                }
            } else {
                for (int p = lane; p < half; p += kWave) {
                    const int i0 = (ROPE == kRopeNeox) ? p : 2 * p;
                    const int i1 = (ROPE == kRopeNeox) ? p + half : 2 * p + 1;
                    float x0 = src[i0];
                    float x1 = src[i1];
                    if (wr) {
                        x0 = (wr[i0] * x0) * r;
                        x1 = (wr[i1] * x1) * r;
                    }
                    float sn, cn;
                    sincos_angle(static_cast<float>(pos) * tab.v[p], &sn, &cn);
                    const f2 y = rope_pair(x0, x1, cn, sn);
                    const float y0 = y.x, y1 = y.y;
                    dst[i0] = y0;
                    dst[i1] = y1;
                    if (kv) {
                        args.kc[at + i0] = f32_to_f16_bits(y0);
                        args.kc[at + i1] = f32_to_f16_bits(y1);
                    }
                }
            }
        }
        __syncthreads();
    }
}

// One float4 per lane, one wave per workgroup: two heads (head_dim 128) of
// one token, 32 lanes per head -- the streaming shape that moves an in-place
// 1-read/1-write array fastest (one float4 per lane, one-wave workgroups;
// a plain in-place stream probe reaches 84% of peak this way against 81% with
// two float4 per lane).  It takes RoPE alone, per-head norm and per-head
// norm -> RoPE (no row norm, no KV store): in-process A/B, p50, configs[4]
// RoPE 54.03 -> 52.19 us, configs[2] QK-norm -> RoPE 28.44 -> 27.12 us.
// The arithmetic is the unit kernel's, operation for operation, so results
// are bit-identical: a NeoX partner (hd/2 away) comes from lane l ^ 16 by a
// swizzle; the per-head sum of squares first adds the two halves of a unit
// in the unit kernel's order (first half + second half), then runs the same
// 16-lane DPP tree.  Q heads come first in the grid, then K heads.
template <int ROPE, int NORM>
__global__ __launch_bounds__(64) void head_stream_kernel(const HeadArgs args, InvFreq tab, int64_t wg_q) {
    constexpr int HD = 128, HALF = 64;
    __shared__ __align__(16) float cs[2 * HALF];
    const int lane = threadIdx.x;
    const int ii = lane & 31;  // float4 of the head: elements [4 ii, 4 ii + 4)
    const int64_t w = blockIdx.x;
    const bool isq = w < wg_q;  // workgroup-uniform
    const int nh = isq ? args.nq : args.nkv;
    const int64_t g = 2 * (isq ? w : w - wg_q) + (lane >> 5);  // head in [tokens][nh]
    const int64_t t = (2 * (isq ? w : w - wg_q)) / nh;         // both heads of the workgroup: one token
    const float* src = isq ? args.qi + g * HD : args.k + g * HD;
    float* dst = isq ? args.qo + g * HD : args.k + g * HD;
    f4 v = ld4<true>(src + 4 * ii);
    f4 wv = f4(1.0f);
    if constexpr (NORM == kNormHead) wv = ld4<false>((isq ? args.wq : args.wk) + 4 * ii);
    if constexpr (ROPE != kRopeNone) {
        const int pos = args.positions ? args.positions[t] : args.pos0 + static_cast<int>(t);
        float sn, cn;
        sincos_angle(static_cast<float>(pos) * tab.v[lane], &sn, &cn);
        cs[lane] = cn;
        cs[HALF + lane] = sn;
    }
    if constexpr (NORM == kNormHead) {
        // the unit kernel's dot4(a) + dot4(b), a the first half, then its 16-lane tree
        const float s = dot4(v);
        const float sp = swz_xor16(s);
        const float u = ii < 16 ? s + sp : sp + s;
        const float tot = group_reduce<16>(u, OpAdd{});
        const float r = head_rscale(tot, static_cast<float>(HD), args.eps);
        v = (wv * v) * r;
    }
    if constexpr (ROPE != kRopeNone) {
        __syncthreads();  // cs
        if constexpr (ROPE == kRopeNeox) {
            f4 o;
            o.x = swz_xor16(v.x), o.y = swz_xor16(v.y), o.z = swz_xor16(v.z), o.w = swz_xor16(v.w);
            const int p = 4 * (ii & 15);
            const f4 c = *reinterpret_cast<const f4*>(cs + p);
            const f4 sn = *reinterpret_cast<const f4*>(cs + HALF + p);
            if (ii < 16) {  // x0 = v, x1 = partner: x0 c - x1 s
                v = f4{rope_pair(v.x, o.x, c.x, sn.x).x, rope_pair(v.y, o.y, c.y, sn.y).x,
                       rope_pair(v.z, o.z, c.z, sn.z).x, rope_pair(v.w, o.w, c.w, sn.w).x};
            } else {  // x0 = partner, x1 = v: x0 s + x1 c
                v = f4{rope_pair(o.x, v.x, c.x, sn.x).y, rope_pair(o.y, v.y, c.y, sn.y).y,
                       rope_pair(o.z, v.z, c.z, sn.z).y, rope_pair(o.w, v.w, c.w, sn.w).y};
            }
        } else {  // interleaved: pairs 2 ii and 2 ii + 1 inside the float4
            const f2 c = *reinterpret_cast<const f2*>(cs + 2 * ii);
            const f2 sn = *reinterpret_cast<const f2*>(cs + HALF + 2 * ii);
            const f2 a0 = rope_pair(v.x, v.y, c.x, sn.x), a1 = rope_pair(v.z, v.w, c.y, sn.y);
            v = f4{a0.x, a0.y, a1.x, a1.y};
        }
    }
    st4<true>(dst + 4 * ii, v);
}

template <int ROPE, int NORM>
int launch_stream(const HeadArgs& a, const InvFreq& tab, hipStream_t s) {
    const int64_t wg_q = a.tokens * a.nq / 2, wg_k = a.tokens * a.nkv / 2;
    return launch(head_stream_kernel<ROPE, NORM>, dim3(static_cast<unsigned>(wg_q + wg_k)), dim3(64), 0, s, a,
                  tab, wg_q);
}

template <int ROPE, int NORM, int G, bool KV>
int dispatch_slots(unsigned grid, unsigned threads, hipStream_t s, const HeadArgs& a, int slots,
                   const InvFreq& tab) {
    if (slots == 1)
        return launch(head_ops_vec_kernel<ROPE, NORM, G, 1, KV>, dim3(grid), dim3(threads), 0, s, a, tab);
    return launch(head_ops_vec_kernel<ROPE, NORM, G, 2, KV>, dim3(grid), dim3(threads), 0, s, a, tab);
}

template <int ROPE, int NORM, bool KV>
int dispatch_vec(int G, unsigned grid, unsigned threads, hipStream_t s, const HeadArgs& a, int slots,
                 const InvFreq& tab) {
    switch (G) {
        case 8: return dispatch_slots<ROPE, NORM, 8, KV>(grid, threads, s, a, slots, tab);
        case 16: return dispatch_slots<ROPE, NORM, 16, KV>(grid, threads, s, a, slots, tab);
        case 32: return dispatch_slots<ROPE, NORM, 32, KV>(grid, threads, s, a, slots, tab);
        default: return FENCE_ERROR_INVALID_VALUE;
    }
}

template <int ROPE, int NORM>
int dispatch(bool vec, int G, unsigned grid, unsigned threads, hipStream_t s, const HeadArgs& a, int hd,
             int slots, const InvFreq& tab) {
    if (!vec) return launch(head_ops_scalar_kernel<ROPE, NORM>, dim3(grid), dim3(256), 0, s, a, hd, tab);
    if constexpr (NORM != kNormRow) {
        if (G == 16 && !a.kc && a.nq % 2 == 0 && a.nkv % 2 == 0 &&
            a.tokens * (a.nq + a.nkv) / 2 * 64 <= kMaxLaunchLanes)  // else the grid-strided unit kernel
            return launch_stream<ROPE, NORM>(a, tab, s);
    }
    if constexpr (ROPE != kRopeNone && NORM != kNormRow) {  // the KV store follows a RoPE
        if (a.kc) return dispatch_vec<ROPE, NORM, true>(G, grid, threads, s, a, slots, tab);
    }
    return dispatch_vec<ROPE, NORM, false>(G, grid, threads, s, a, slots, tab);
}

template <int ROPE>
int dispatch_norm(int norm, bool vec, int G, unsigned grid, unsigned threads, hipStream_t s, const HeadArgs& a,
                  int hd, int slots, const InvFreq& tab) {
    switch (norm) {
        case kNormNone: return dispatch<ROPE, kNormNone>(vec, G, grid, threads, s, a, hd, slots, tab);
        case kNormRow: return dispatch<ROPE, kNormRow>(vec, G, grid, threads, s, a, hd, slots, tab);
        case kNormHead: return dispatch<ROPE, kNormHead>(vec, G, grid, threads, s, a, hd, slots, tab);
        default: return FENCE_ERROR_INVALID_VALUE;
    }
}

bool ok4(const void* p) { return p == nullptr || aligned(p, 4); }
bool ok16(const void* p) { return p == nullptr || aligned(p, 16); }

}  // namespace

// Host computation of the reference's per-pair frequency (ops.cuh:133).
// A one-entry cache per host thread avoids recomputing hd/2 powf calls for
// every decode step with the same (base, head_dim).
void rope_inv_freq_host(float* out, int hd, float base) {
    thread_local int c_hd = -1;
    thread_local uint32_t c_base_bits = 0;
    thread_local float c_vals[kMaxHalf];
    const uint32_t bits = __builtin_bit_cast(uint32_t, base);
    if (c_hd != hd || c_base_bits != bits) {
        for (int p = 0; p < hd / 2; ++p)
            c_vals[p] = 1.0f / powf(base, static_cast<float>(2 * p) / static_cast<float>(hd));
        c_hd = hd;
        c_base_bits = bits;
    }
    for (int p = 0; p < hd / 2; ++p) out[p] = c_vals[p];
}

// Shared entry for every head-structured op.
//   qo/qi: q output/input [tokens][nq][hd] (equal for the in-place forms)
//   k:     [tokens][nkv][hd], in place
//   norm:  none | row (q row, weight wq[nq*hd]) | head (wq[hd], wk[hd])
//   kv:    optional KV store (kc, vc, v, max_ctx; see HeadArgs), with a RoPE
//          and without the row norm
int head_ops_launch(float* qo, const float* qi, float* k, const float* wq, const float* wk,
                    int64_t tokens, int nq, int nkv, int hd, float eps, const int32_t* positions,
                    int pos0, float base, int rope, int norm, hipStream_t s, uint16_t* kc = nullptr,
                    uint16_t* vc = nullptr, const float* v = nullptr, int max_ctx = 0) {
    if (tokens < 0 || nq < 0 || nkv < 0 || hd <= 0) return FENCE_ERROR_INVALID_VALUE;
    if (rope != kRopeNone && rope != kRopeNeox && rope != kRopeInter) return FENCE_ERROR_INVALID_VALUE;
    if (nq > 0 && (!qo || !qi)) return FENCE_ERROR_INVALID_VALUE;
    if (nkv > 0 && !k) return FENCE_ERROR_INVALID_VALUE;
    if (norm == kNormRow && nq > 0 && !wq) return FENCE_ERROR_INVALID_VALUE;
    if (norm == kNormHead && ((nq > 0 && !wq) || (nkv > 0 && !wk))) return FENCE_ERROR_INVALID_VALUE;
    if (rope != kRopeNone) {
        if (hd % 2 != 0 || hd > 2 * kMaxHalf) return FENCE_ERROR_INVALID_VALUE;
        if (!(base > 0.0f) || !std::isfinite(base)) return FENCE_ERROR_INVALID_VALUE;
    }
    if (!ok4(qo) || !ok4(qi) || !ok4(k) || !ok4(wq) || !ok4(wk) || !ok4(positions))
        return FENCE_ERROR_INVALID_VALUE;
    if (kc) {
        if (!vc || !v || nkv <= 0 || max_ctx <= 0 || rope == kRopeNone || norm == kNormRow) return FENCE_ERROR_INVALID_VALUE;
        if (!aligned(kc, 2) || !aligned(vc, 2) || !ok4(v)) return FENCE_ERROR_INVALID_VALUE;
        // positions from pos0 are checked here; device positions by the kernel
        if (!positions && (pos0 < 0 || static_cast<int64_t>(pos0) + tokens > max_ctx)) return FENCE_ERROR_INVALID_VALUE;
    }
    if (tokens == 0 || nq + nkv == 0) return FENCE_SUCCESS;
    if (nq == 0) {  // keep q pointers valid for address arithmetic only
        qo = k;
        qi = k;
    }
    if (nkv == 0) k = qo;

    InvFreq tab{};
    if (rope != kRopeNone) rope_inv_freq_host(tab.v, hd, base);

    const int G = hd / 8;
    bool vec = (hd == 64 || hd == 128 || hd == 256) && ok16(qo) && ok16(qi) && ok16(k) &&
               ok16(wq) && ok16(wk) && ok16(kc) && ok16(vc) && ok16(v);
    unsigned threads = 256;
    int slots = 0;
    // Units per lane: RoPE alone streams best with one (two float4 per lane:
    // 8192 tokens x 40 heads, p50 54.75 -> 53.99 us, in-process A/B); with a
    // norm two, which halve the lanes that reduce (QK-norm -> RoPE at 4096
    // tokens 28.44 us with two, 30.20 with one).  plan_row halves the target
    // anyway when the tokens cannot fill the GPU.
    const int target = norm == kNormNone ? 1 : FENCE_HEAD_SLOTS;
    if (vec) vec = plan_row(tokens, static_cast<int64_t>(nq + nkv) * G, target, 2, &threads, &slots);
    const unsigned grid = grid_1d(tokens, 1, 1 << 20);
    const HeadArgs a{qo, qi, k, wq, wk, tokens, nq, nkv, eps, positions, pos0, kc, vc, v, max_ctx};
    switch (rope) {
        case kRopeNone: return dispatch_norm<kRopeNone>(norm, vec, G, grid, threads, s, a, hd, slots, tab);
        case kRopeNeox: return dispatch_norm<kRopeNeox>(norm, vec, G, grid, threads, s, a, hd, slots, tab);
        default: return dispatch_norm<kRopeInter>(norm, vec, G, grid, threads, s, a, hd, slots, tab);
    }
}

}  // namespace fence

using fence::head_ops_launch;

extern "C" int fence_rms_norm_per_head(float* x, const float* w, int n_heads, int head_dim,
                                       float eps, hipStream_t stream) {
    if (!w) return FENCE_ERROR_INVALID_VALUE;
    return head_ops_launch(x, x, nullptr, w, nullptr, 1, n_heads, 0, head_dim, eps, nullptr, 0,
                           1.0f, fence::kRopeNone, fence::kNormHead, stream);
}

extern "C" int fence_apply_rope(float* q, float* k, int head_dim, int n_q_heads, int n_kv_heads,
                                int pos, float freq_base, hipStream_t stream) {
    return head_ops_launch(q, q, k, nullptr, nullptr, 1, n_q_heads, n_kv_heads, head_dim, 0.0f,
                           nullptr, pos, freq_base, fence::kRopeNeox, fence::kNormNone, stream);
}

extern "C" int fence_rope(float* q, float* k, int64_t tokens, int n_q_heads, int n_kv_heads,
                          int head_dim, const int32_t* positions, int pos0, float freq_base,
                          int style, hipStream_t stream) {
    if (style != FENCE_ROPE_NEOX && style != FENCE_ROPE_INTERLEAVED) return FENCE_ERROR_INVALID_VALUE;
    return head_ops_launch(q, q, k, nullptr, nullptr, tokens, n_q_heads, n_kv_heads, head_dim, 0.0f,
                           positions, pos0, freq_base, style, fence::kNormNone, stream);
}

extern "C" int fence_qk_norm_rope(float* q, float* k, const float* q_norm_w, const float* k_norm_w,
                                  int64_t tokens, int n_q_heads, int n_kv_heads, int head_dim,
                                  float eps, const int32_t* positions, int pos0, float freq_base,
                                  int style, hipStream_t stream) {
    if (style != FENCE_ROPE_NEOX && style != FENCE_ROPE_INTERLEAVED) return FENCE_ERROR_INVALID_VALUE;
    return head_ops_launch(q, q, k, q_norm_w, k_norm_w, tokens, n_q_heads, n_kv_heads, head_dim,
                           eps, positions, pos0, freq_base, style, fence::kNormHead, stream);
}

extern "C" int fence_qk_norm_rope_store_kv(float* q, float* k, const float* v, const float* q_norm_w,
                                           const float* k_norm_w, void* k_cache, void* v_cache, int max_ctx,
                                           int64_t tokens, int n_q_heads, int n_kv_heads, int head_dim,
                                           float eps, const int32_t* positions, int pos0, float freq_base,
                                           int style, hipStream_t stream) {
    if (style != FENCE_ROPE_NEOX && style != FENCE_ROPE_INTERLEAVED) return FENCE_ERROR_INVALID_VALUE;
    if (!k_cache || (q_norm_w == nullptr) != (k_norm_w == nullptr)) return FENCE_ERROR_INVALID_VALUE;
    return head_ops_launch(q, q, k, q_norm_w, k_norm_w, tokens, n_q_heads, n_kv_heads, head_dim, eps, positions,
                           pos0, freq_base, style, q_norm_w ? fence::kNormHead : fence::kNormNone, stream,
                           static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), v, max_ctx);
}

extern "C" int fence_rms_norm_rope(float* out, const float* x, const float* w, float* k,
                                   int64_t tokens, int n_q_heads, int n_kv_heads, int head_dim,
                                   float eps, const int32_t* positions, int pos0, float freq_base,
                                   int style, hipStream_t stream) {
    if (style != FENCE_ROPE_NEOX && style != FENCE_ROPE_INTERLEAVED) return FENCE_ERROR_INVALID_VALUE;
    if (n_q_heads <= 0 || !w) return FENCE_ERROR_INVALID_VALUE;
    return head_ops_launch(out, x, k, w, nullptr, tokens, n_q_heads, n_kv_heads, head_dim, eps,
                           positions, pos0, freq_base, style, fence::kNormRow, stream);
}

extern "C" int fence_rope_inv_freq(float* inv_freq, int head_dim, float freq_base) {
    if (!inv_freq || head_dim <= 0 || head_dim % 2 != 0 || head_dim > 2 * fence::kMaxHalf)
        return FENCE_ERROR_INVALID_VALUE;
    fence::rope_inv_freq_host(inv_freq, head_dim, freq_base);
    return FENCE_SUCCESS;
}
