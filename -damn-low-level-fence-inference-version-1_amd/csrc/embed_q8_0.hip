// embed_q8_0.hip -- Q8_0 embedding dequant-gather (optionally fused with
// RMSNorm) on gfx950.
//
// Follows embed_q8_0, src/kernels/gemv_q8_0.cuh:12-36, on the block layout of
// src/kernels/q8_0_types.h:8-17 (fp16 scale d, then 32 int8 qs; 34 bytes):
//   out[i] = float(d[i/32]) * float(qs[i/32][i%32])
// An 11-bit by 8-bit significand product fits fp32 exactly, so every output
// is bit-identical to the reference formula.
//
// Each lane produces one float4 of output: block b = f/8 of the row, quarter
// k = f%8.  It reads the block's fp16 scale and its four int8s with 2-byte
// loads straight from global memory (the 34-byte blocks are only 2-byte
// aligned; eight neighbouring lanes share a block, so the loads coalesce into
// the same cache lines), converts in registers and writes a 128-bit
// non-temporal store.  The plain gather runs a 2-D grid (token x row chunk of
// 256 float4s) with no LDS and no barrier; the fused form runs one workgroup
// per token, keeps the row in VGPRs, reduces the sum of squares and applies
// rms_norm (src/kernels/ops.cuh:40-44) before the single write.
#include "common.hpp"

// Fused gather->norm: float4s per lane, and workgroups per CU in its grid
// (each workgroup loops over tokens with its weights loaded once).  Measured
// on configs[3] (8192 Zipf ids x 5120, in-process A/B): 4 per CU x 4 float4
// 30.5 us (75% of HBM peak); 2 x 2 32.6 us; 2 x 4 38.5 us; one workgroup per
// token 39 us.
#ifndef FENCE_GATHER_RMS_VPT
#define FENCE_GATHER_RMS_VPT 4
#endif
#ifndef FENCE_GATHER_RMS_WG_PER_CU
#define FENCE_GATHER_RMS_WG_PER_CU 4
#endif

namespace fence {
namespace {

constexpr int kChunk = 256;        // float4 outputs per workgroup in the plain gather
constexpr int kMaxDimVec = 16384;  // fused form: up to 4 float4 per lane at 1024 lanes

// The raw bits behind one float4 of a dequantised row: the block's fp16
// scale and the four int8 of quarter f%8.  BYTES: table only 1-byte aligned.
struct Q8Bits {
    uint32_t d;
    uint32_t q;
};

template <bool BYTES>
__device__ __forceinline__ Q8Bits load_q8(const uint8_t* row, int f) {
    const uint8_t* blk = row + 34 * (f >> 3);
    const int k = f & 7;
    Q8Bits r;
    if constexpr (BYTES) {
        const uint8_t* p = blk + 2 + 4 * k;
        r.d = static_cast<uint32_t>(blk[0]) | (static_cast<uint32_t>(blk[1]) << 8);
        r.q = static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) |
              (static_cast<uint32_t>(p[2]) << 16) | (static_cast<uint32_t>(p[3]) << 24);
    } else {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(blk);
        r.d = h[0];
        r.q = static_cast<uint32_t>(h[1 + 2 * k]) | (static_cast<uint32_t>(h[2 + 2 * k]) << 16);
    }
    return r;
}

__device__ __forceinline__ f4 dequant_bits(Q8Bits b) {
    const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b.d)));
    f4 v;
    v.x = d * static_cast<float>(static_cast<int8_t>(b.q & 0xFFu));
    v.y = d * static_cast<float>(static_cast<int8_t>((b.q >> 8) & 0xFFu));
    v.z = d * static_cast<float>(static_cast<int8_t>((b.q >> 16) & 0xFFu));
    v.w = d * static_cast<float>(static_cast<int8_t>(b.q >> 24));
    return v;
}

template <bool BYTES>
__device__ __forceinline__ f4 dequant4(const uint8_t* row, int f) {
    return dequant_bits(load_q8<BYTES>(row, f));
}

template <bool VEC_OUT>
__device__ __forceinline__ void store4(float* p, f4 v) {
    if constexpr (VEC_OUT) {
        st4<true>(p, v);
    } else {
        p[0] = v.x;
        p[1] = v.y;
        p[2] = v.z;
        p[3] = v.w;
    }
}

__device__ __forceinline__ int64_t token_id(const int32_t* ids, int single_id, int64_t t) {
    return ids ? static_cast<int64_t>(ids[t]) : static_cast<int64_t>(single_id);
}

// grid.x = tokens (grid-stride), grid.y = row chunks of kChunk float4s.
template <bool BYTES, bool VEC_OUT>
__global__ __launch_bounds__(kChunk) void q8_gather_kernel(float* out, const uint8_t* table,
                                                           int64_t vocab, const int32_t* ids,
                                                           int single_id, int64_t tokens, int dim) {
    const int dim4 = dim >> 2;
    const int f = blockIdx.y * kChunk + threadIdx.x;
    if (f >= dim4) return;
    const int64_t rb = static_cast<int64_t>(dim / 32) * 34;
    for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
        const int64_t id = token_id(ids, single_id, t);
        f4 v;
        if (id < 0 || id >= vocab) v = f4(__builtin_nanf(""));
        else v = dequant4<BYTES>(table + id * rb, f);
        store4<VEC_OUT>(out + t * dim + 4 * f, v);
    }
}

// One workgroup per token; `vpt` float4s per lane.
template <bool BYTES, int MAXV>
__global__ __launch_bounds__(1024) void q8_gather_rms_kernel(float* out, const uint8_t* table,
                                                             int64_t vocab, const int32_t* ids,
                                                             int64_t tokens, int dim, const float* w,
                                                             float eps, int vpt) {
    __shared__ float red[16];
    const int T = blockDim.x;
    const int dim4 = dim >> 2;
    const int64_t rb = static_cast<int64_t>(dim / 32) * 34;
    f4 wv[MAXV];  // the weights: the same for every token, loaded once
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
        const int f = threadIdx.x + j * T;
        wv[j] = (j < vpt && f < dim4) ? ld4<false>(w + 4 * f) : f4(0.0f);
    }
    for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
        const int64_t id = ids[t];
        float* orow = out + t * dim;
        const bool ok = id >= 0 && id < vocab;  // uniform across the workgroup
        const uint8_t* row = table + (ok ? id : 0) * rb;
        Q8Bits bits[MAXV];
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {  // every load of the lane first
            const int f = threadIdx.x + j * T;
            bits[j] = Q8Bits{0u, 0u};
            if (ok && j < vpt && f < dim4) bits[j] = load_q8<BYTES>(row, f);
        }
        f4 v[MAXV];
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            v[j] = dequant_bits(bits[j]);  // zero bits give +0
            ss += dot4(v[j]);
        }
        const float tot = block_reduce_dyn(ss, OpAdd(), red);
        const float rs = rsqrtf(tot / static_cast<float>(dim) + eps);
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int f = threadIdx.x + j * T;
            if (j < vpt && f < dim4) {
                const f4 o = ok ? (wv[j] * v[j]) * rs : f4(__builtin_nanf(""));
                st4<true>(orow + 4 * f, o);
            }
        }
        __syncthreads();  // red[] is rewritten for the next token
    }
}

// Any alignment of out / w and dim % 32 == 0: one lane per Q8_0 block,
// scalar stores; reads the row twice.
__global__ __launch_bounds__(256) void q8_gather_rms_scalar_kernel(
    float* out, const uint8_t* table, int64_t vocab, const int32_t* ids, int64_t tokens, int dim,
    const float* w, float eps) {
    __shared__ float red[4];
    const int nb = dim / 32;
    for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
        const int64_t id = ids[t];
        float* orow = out + t * dim;
        if (id < 0 || id >= vocab) {
            for (int i = threadIdx.x; i < dim; i += 256) orow[i] = __builtin_nanf("");
            continue;
        }
        const uint8_t* row = table + id * static_cast<int64_t>(nb) * 34;
        float ss = 0.0f;
        for (int b = threadIdx.x; b < nb; b += 256) {
            for (int q = 0; q < 8; ++q) ss += dot4(dequant4<true>(row, 8 * b + q));
        }
        const float rs = rsqrtf(block_reduce<4>(ss, OpAdd(), red) / static_cast<float>(dim) + eps);
        for (int b = threadIdx.x; b < nb; b += 256) {
            for (int q = 0; q < 8; ++q) {
                const f4 v = dequant4<true>(row, 8 * b + q);
                const int e = 32 * b + 4 * q;
                orow[e + 0] = (w[e + 0] * v.x) * rs;
                orow[e + 1] = (w[e + 1] * v.y) * rs;
                orow[e + 2] = (w[e + 2] * v.z) * rs;
                orow[e + 3] = (w[e + 3] * v.w) * rs;
            }
        }
        __syncthreads();
    }
}

int check_common(float* out, const void* table, int64_t tokens, int dim, int64_t vocab,
                 const int32_t* ids) {
    if (!out || !table || tokens < 0 || dim <= 0 || dim % 32 != 0 || vocab <= 0)
        return FENCE_ERROR_INVALID_VALUE;
    if (!aligned(out, 4) || (ids && !aligned(ids, 4))) return FENCE_ERROR_INVALID_VALUE;
    return FENCE_SUCCESS;
}

int gather_launch(float* out, const void* table_v, int64_t vocab, const int32_t* ids, int single_id,
                  int64_t tokens, int dim, hipStream_t s) {
    const int st = check_common(out, table_v, tokens, dim, vocab, ids);
    if (st || tokens == 0) return st;
    const uint8_t* table = static_cast<const uint8_t*>(table_v);
    const unsigned chunks = static_cast<unsigned>((dim / 4 + kChunk - 1) / kChunk);
    const dim3 grid(grid_1d(tokens, 1, 1 << 20), chunks);
    const bool bytes = !aligned(table, 2);
    const bool vec_out = aligned(out, 16);
    if (bytes) {
        if (vec_out)
            return launch(q8_gather_kernel<true, true>, grid, dim3(kChunk), 0, s, out, table, vocab, ids,
                          single_id, tokens, dim);
        return launch(q8_gather_kernel<true, false>, grid, dim3(kChunk), 0, s, out, table, vocab, ids,
                      single_id, tokens, dim);
    }
    if (vec_out)
        return launch(q8_gather_kernel<false, true>, grid, dim3(kChunk), 0, s, out, table, vocab, ids,
                      single_id, tokens, dim);
    return launch(q8_gather_kernel<false, false>, grid, dim3(kChunk), 0, s, out, table, vocab, ids,
                  single_id, tokens, dim);
}

template <bool BYTES>
int gather_rms_vec(float* out, const uint8_t* table, int64_t vocab, const int32_t* ids,
                   int64_t tokens, int dim, const float* w, float eps, unsigned threads, int vpt,
                   hipStream_t s) {
    const unsigned grid = grid_1d(tokens, 1, 256 * FENCE_GATHER_RMS_WG_PER_CU);
    if (vpt <= 2)
        return launch(q8_gather_rms_kernel<BYTES, 2>, dim3(grid), dim3(threads), 0, s, out, table,
                      vocab, ids, tokens, dim, w, eps, vpt);
    return launch(q8_gather_rms_kernel<BYTES, 4>, dim3(grid), dim3(threads), 0, s, out, table, vocab,
                  ids, tokens, dim, w, eps, vpt);
}

int gather_rms_launch(float* out, const void* table_v, int64_t vocab, const int32_t* ids,
                      int64_t tokens, int dim, const float* w, float eps, hipStream_t s) {
    const int st = check_common(out, table_v, tokens, dim, vocab, ids);
    if (st) return st;
    if (!w || !aligned(w, 4) || (!ids && tokens > 0)) return FENCE_ERROR_INVALID_VALUE;
    if (tokens == 0) return FENCE_SUCCESS;
    const uint8_t* table = static_cast<const uint8_t*>(table_v);
    unsigned threads = 0;
    int vpt = 0;
    const bool vec = dim <= kMaxDimVec && aligned(out, 16) && aligned(w, 16) &&
                     plan_row(tokens, dim / 4, FENCE_GATHER_RMS_VPT, 4, &threads, &vpt);
    if (vec) {
        if (!aligned(table, 2))
            return gather_rms_vec<true>(out, table, vocab, ids, tokens, dim, w, eps, threads, vpt, s);
        return gather_rms_vec<false>(out, table, vocab, ids, tokens, dim, w, eps, threads, vpt, s);
    }
    const unsigned grid = grid_1d(tokens, 1, 1 << 20);
    return launch(q8_gather_rms_scalar_kernel, dim3(grid), dim3(256), 0, s, out, table, vocab, ids,
                  tokens, dim, w, eps);
}

}  // namespace
}  // namespace fence

extern "C" int fence_embed_q8_0(float* out, const void* weight, int token_id, int dim,
                                hipStream_t stream) {
    if (token_id < 0) return FENCE_ERROR_INVALID_VALUE;
    // The reference signature carries no vocab size: the row is trusted.
    return fence::gather_launch(out, weight, INT64_MAX, nullptr, token_id, 1, dim, stream);
}

extern "C" int fence_embed_q8_0_gather(float* out, const void* table, int64_t vocab,
                                       const int32_t* ids, int64_t tokens, int dim,
                                       hipStream_t stream) {
    if (!ids && tokens > 0) return FENCE_ERROR_INVALID_VALUE;
    return fence::gather_launch(out, table, vocab, ids, 0, tokens, dim, stream);
}

extern "C" int fence_embed_q8_0_gather_rms_norm(float* out, const void* table, int64_t vocab,
                                                const int32_t* ids, int64_t tokens, int dim,
                                                const float* w, float eps, hipStream_t stream) {
    return fence::gather_rms_launch(out, table, vocab, ids, tokens, dim, w, eps, stream);
}
