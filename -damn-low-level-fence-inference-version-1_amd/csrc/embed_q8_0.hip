// embed_q8_0.hip -- Q8_0 embedding dequant-gather (optionally fused with
// RMSNorm) on gfx950.
//
// Follows embed_q8_0, src/kernels/gemv_q8_0.cuh:12-36, on the block layout of
// src/kernels/q8_0_types.h:8-17 (fp16 scale d, then 32 int8 qs; 34 bytes):
//   out[i] = float(d[i/32]) * float(qs[i/32][i%32])
// An 11-bit by 8-bit significand product fits fp32 exactly, so every output
// is bit-identical to the reference formula.
//
// One workgroup per token: the token's row (dim/32 * 34 bytes) is copied to
// LDS with 128-bit loads (rows are 16-byte aligned whenever dim % 256 == 0),
// then each lane builds float4 outputs from one fp16 scale and four int8s
// read out of LDS and writes them with coalesced 128-bit stores.  The fused
// form keeps the row in VGPRs, reduces the sum of squares and applies
// rms_norm (src/kernels/ops.cuh:40-44) before the single write.
#include "common.hpp"

namespace fence {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxDimVec = 16384;  // 16 float4 per lane

enum { kStage16 = 16, kStage2 = 2, kStage1 = 1 };

__device__ __forceinline__ f4 dequant4(const uint8_t* lds_row, int f) {
    // float4 f covers elements 4f..4f+3: block b = f/8, quarter k = f%8
    const int b = f >> 3;
    const int k = f & 7;
    const uint8_t* blk = lds_row + 34 * b;
    const uint16_t dbits = *reinterpret_cast<const uint16_t*>(blk);
    const uint32_t lo = *reinterpret_cast<const uint16_t*>(blk + 2 + 4 * k);
    const uint32_t hi = *reinterpret_cast<const uint16_t*>(blk + 4 + 4 * k);
    const uint32_t q = lo | (hi << 16);
    const float d = static_cast<float>(__builtin_bit_cast(_Float16, dbits));
    f4 v;
    v.x = d * static_cast<float>(static_cast<int8_t>(q & 0xFFu));
    v.y = d * static_cast<float>(static_cast<int8_t>((q >> 8) & 0xFFu));
    v.z = d * static_cast<float>(static_cast<int8_t>((q >> 16) & 0xFFu));
    v.w = d * static_cast<float>(static_cast<int8_t>(q >> 24));
    return v;
}

template <bool NORM, int MAXV>
__global__ __launch_bounds__(kThreads) void q8_gather_vec_kernel(
    float* out, const uint8_t* table, int64_t vocab, const int32_t* ids, int single_id,
    int64_t tokens, int dim, const float* w, float eps, int vpt, int stage) {
    extern __shared__ __align__(16) uint8_t row_lds[];
    __shared__ float red[kThreads / kWave];
    const int rb = (dim / 32) * 34;
    const int dim4 = dim / 4;
    for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
        const int64_t id = ids ? static_cast<int64_t>(ids[t]) : static_cast<int64_t>(single_id);
        float* orow = out + t * dim;
        if (id < 0 || id >= vocab) {  // uniform: the whole workgroup takes it
            const f4 qnan = f4(__builtin_nanf(""));
#pragma unroll
            for (int j = 0; j < MAXV; ++j) {
                const int f = threadIdx.x + j * kThreads;
                if (j < vpt && f < dim4) st4<true>(orow + 4 * f, qnan);
            }
            continue;
        }
        const uint8_t* src = table + id * rb;
        if (stage == kStage16) {
            for (int c = threadIdx.x; c < rb / 16; c += kThreads)
                *reinterpret_cast<u4*>(row_lds + 16 * c) =
                    __builtin_nontemporal_load(reinterpret_cast<const u4*>(src) + c);
        } else if (stage == kStage2) {
            for (int c = threadIdx.x; c < rb / 2; c += kThreads)
                reinterpret_cast<uint16_t*>(row_lds)[c] = reinterpret_cast<const uint16_t*>(src)[c];
        } else {
            for (int c = threadIdx.x; c < rb; c += kThreads) row_lds[c] = src[c];
        }
        __syncthreads();

        f4 v[MAXV];
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int f = threadIdx.x + j * kThreads;
            if (j < vpt && f < dim4) {
                v[j] = dequant4(row_lds, f);
                if constexpr (NORM) ss += dot4(v[j]);
            }
        }
        float rs = 1.0f;
        if constexpr (NORM) {
            const float tot = block_reduce<kThreads / kWave>(ss, OpAdd(), red);
            rs = rsqrtf(tot / static_cast<float>(dim) + eps);
        }
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int f = threadIdx.x + j * kThreads;
            if (j < vpt && f < dim4) {
                f4 o = v[j];
                if constexpr (NORM) o = (ld4<false>(w + 4 * f) * o) * rs;
                st4<true>(orow + 4 * f, o);
            }
        }
        __syncthreads();  // row_lds and red[] are rewritten for the next token
    }
}

// Any alignment and dim % 32 == 0: one lane per Q8_0 block, byte reads from
// global memory, scalar stores.  The fused form reads the row twice.
template <bool NORM>
__global__ __launch_bounds__(kThreads) void q8_gather_scalar_kernel(
    float* out, const uint8_t* table, int64_t vocab, const int32_t* ids, int single_id,
    int64_t tokens, int dim, const float* w, float eps) {
    __shared__ float red[kThreads / kWave];
    const int nb = dim / 32;
    for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
        const int64_t id = ids ? static_cast<int64_t>(ids[t]) : static_cast<int64_t>(single_id);
        float* orow = out + t * dim;
        if (id < 0 || id >= vocab) {
            for (int i = threadIdx.x; i < dim; i += kThreads) orow[i] = __builtin_nanf("");
            continue;
        }
        const uint8_t* row = table + id * static_cast<int64_t>(nb) * 34;
        float rs = 1.0f;
        if constexpr (NORM) {
            float ss = 0.0f;
            for (int b = threadIdx.x; b < nb; b += kThreads) {
                const uint8_t* blk = row + 34 * b;
                const float d = static_cast<float>(
                    __builtin_bit_cast(_Float16, static_cast<uint16_t>(blk[0] | (blk[1] << 8))));
                for (int i = 0; i < 32; ++i) {
                    const float v = d * static_cast<float>(static_cast<int8_t>(blk[2 + i]));
                    ss += v * v;
                }
            }
            rs = rsqrtf(block_reduce<kThreads / kWave>(ss, OpAdd(), red) / static_cast<float>(dim) + eps);
        }
        for (int b = threadIdx.x; b < nb; b += kThreads) {
            const uint8_t* blk = row + 34 * b;
            const float d = static_cast<float>(
                __builtin_bit_cast(_Float16, static_cast<uint16_t>(blk[0] | (blk[1] << 8))));
            for (int i = 0; i < 32; ++i) {
                float v = d * static_cast<float>(static_cast<int8_t>(blk[2 + i]));
                if constexpr (NORM) v = (w[32 * b + i] * v) * rs;
                orow[32 * b + i] = v;
            }
        }
        __syncthreads();
    }
}

template <bool NORM, int MAXV>
int vec_launch(float* out, const uint8_t* table, int64_t vocab, const int32_t* ids, int single_id,
               int64_t tokens, int dim, const float* w, float eps, int vpt, int stage,
               hipStream_t s) {
    const unsigned grid = grid_1d(tokens, 1, 1 << 20);
    const size_t lds = ((static_cast<size_t>(dim / 32) * 34) + 15) & ~size_t(15);
    return launch(q8_gather_vec_kernel<NORM, MAXV>, dim3(grid), dim3(kThreads), lds, s, out, table,
                  vocab, ids, single_id, tokens, dim, w, eps, vpt, stage);
}

template <bool NORM>
int gather_launch(float* out, const void* table_v, int64_t vocab, const int32_t* ids,
                  int single_id, int64_t tokens, int dim, const float* w, float eps,
                  hipStream_t s) {
    const uint8_t* table = static_cast<const uint8_t*>(table_v);
    if (!out || !table || tokens < 0 || dim <= 0 || dim % 32 != 0 || vocab <= 0)
        return FENCE_ERROR_INVALID_VALUE;
    if (NORM && !w) return FENCE_ERROR_INVALID_VALUE;
    if (!aligned(out, 4) || (w && !aligned(w, 4)) || (ids && !aligned(ids, 4)))
        return FENCE_ERROR_INVALID_VALUE;
    if (tokens == 0) return FENCE_SUCCESS;
    const int rb = (dim / 32) * 34;
    const bool vec = dim <= kMaxDimVec && aligned(out, 16) && (!NORM || aligned(w, 16));
    if (vec) {
        int stage = kStage1;
        if (aligned(table, 16) && rb % 16 == 0) stage = kStage16;
        else if (aligned(table, 2)) stage = kStage2;
        const int dim4 = dim / 4;
        const int vpt = (dim4 + kThreads - 1) / kThreads;
        if (vpt <= 4) return vec_launch<NORM, 4>(out, table, vocab, ids, single_id, tokens, dim, w, eps, vpt, stage, s);
        if (vpt <= 8) return vec_launch<NORM, 8>(out, table, vocab, ids, single_id, tokens, dim, w, eps, vpt, stage, s);
        return vec_launch<NORM, 16>(out, table, vocab, ids, single_id, tokens, dim, w, eps, vpt, stage, s);
    }
    const unsigned grid = grid_1d(tokens, 1, 1 << 20);
    return launch(q8_gather_scalar_kernel<NORM>, dim3(grid), dim3(kThreads), 0, s, out, table, vocab,
                  ids, single_id, tokens, dim, w, eps);
}

}  // namespace
}  // namespace fence

extern "C" int fence_embed_q8_0(float* out, const void* weight, int token_id, int dim,
                                hipStream_t stream) {
    if (token_id < 0) return FENCE_ERROR_INVALID_VALUE;
    // The reference signature carries no vocab size: the row is trusted.
    return fence::gather_launch<false>(out, weight, INT64_MAX, nullptr, token_id, 1, dim, nullptr,
                                       0.0f, stream);
}

extern "C" int fence_embed_q8_0_gather(float* out, const void* table, int64_t vocab,
                                       const int32_t* ids, int64_t tokens, int dim,
                                       hipStream_t stream) {
    if (!ids && tokens > 0) return FENCE_ERROR_INVALID_VALUE;
    return fence::gather_launch<false>(out, table, vocab, ids, 0, tokens, dim, nullptr, 0.0f, stream);
}

extern "C" int fence_embed_q8_0_gather_rms_norm(float* out, const void* table, int64_t vocab,
                                                const int32_t* ids, int64_t tokens, int dim,
                                                const float* w, float eps, hipStream_t stream) {
    if (!ids && tokens > 0) return FENCE_ERROR_INVALID_VALUE;
    return fence::gather_launch<true>(out, table, vocab, ids, 0, tokens, dim, w, eps, stream);
}
