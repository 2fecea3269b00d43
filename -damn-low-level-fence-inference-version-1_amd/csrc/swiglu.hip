// swiglu.hip -- out = silu(gate) * up on gfx950, in fp32 and/or rounded to
// binary16 for the next GEMV's input.
//
// Follows silu_elementwise_mul, src/kernels/ops.cuh:183-202:
//   out[i] = (g / (1.0f + expf(-g))) * up[i],  g = gate[i].
// Streaming kernel: one float4 of gate and one of up per lane, non-temporal
// 128-bit loads and stores, one-wave workgroups.  Measured on MI355X, more
// float4s per lane (a deeper unroll) lowers the achieved bandwidth -- 8 per
// lane per stream halves it -- while many shallow waves reach 72% of peak at
// 29 MB per stream and 82% at 470 MB with 256-thread workgroups, 84% with
// 64-thread ones (in-process A/B, p50: 8192 x 14336 216.5 -> 209.9 us,
// 4096 x 12288 93.9 -> 90.3 us, 512 x 14336 15.8 -> 15.3 us; a plain
// 2-read/1-write stream probe: 82.4% at 256 threads, 84.6% at 128, 84.8% at 64).
// out may alias gate or up: each element is read and written by the same
// lane, reads first.
#include "common.hpp"

namespace fence {
namespace {

constexpr int kSwigluThreads = 64;
constexpr int kSwigluUnroll = 1;

// OUT32: fp32 result to `out`; OUT16: its binary16 rounding to `out16`
// (the f32_to_f16 that src/model/qwen3.cu:336 runs as a separate pass).
template <int UNROLL, bool OUT32, bool OUT16>
__global__ __launch_bounds__(kSwigluThreads) void swiglu_vec_kernel(
    float* out, uint16_t* out16, const float* gate, const float* up, int64_t n4) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * (kSwigluThreads * UNROLL) + threadIdx.x;
    f4 g[UNROLL], u[UNROLL];
#pragma unroll
    for (int j = 0; j < UNROLL; ++j) {
        const int64_t i = base + static_cast<int64_t>(j) * kSwigluThreads;
        if (i < n4) {
            g[j] = ld4<true>(gate + 4 * i);
            u[j] = ld4<true>(up + 4 * i);
        }
    }
#pragma unroll
    for (int j = 0; j < UNROLL; ++j) {
        const int64_t i = base + static_cast<int64_t>(j) * kSwigluThreads;
        if (i < n4) {
            f4 r;
            r.x = silu_mul(g[j].x, u[j].x);
            r.y = silu_mul(g[j].y, u[j].y);
            r.z = silu_mul(g[j].z, u[j].z);
            r.w = silu_mul(g[j].w, u[j].w);
            if constexpr (OUT32) st4<true>(out + 4 * i, r);
            if constexpr (OUT16) st_h4<true>(out16 + 4 * i, r);
        }
    }
}

// Scalar form for unaligned pointers and the n % 4 tail; out or out16 may be null.
__global__ __launch_bounds__(kSwigluThreads) void swiglu_scalar_kernel(
    float* out, uint16_t* out16, const float* gate, const float* up, int64_t begin, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kSwigluThreads;
    for (int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kSwigluThreads + threadIdx.x; i < n;
         i += stride) {
        const float r = silu_mul(gate[i], up[i]);
        if (out) out[i] = r;
        if (out16) out16[i] = f32_to_f16_bits(r);
    }
}

template <bool OUT32, bool OUT16>
int launch_swiglu_vec(unsigned grid, hipStream_t s, float* out, uint16_t* out16, const float* gate,
                      const float* up, int64_t n4) {
    return launch(swiglu_vec_kernel<kSwigluUnroll, OUT32, OUT16>, dim3(grid), dim3(kSwigluThreads), 0, s,
                  out, out16, gate, up, n4);
}

// out or out16 may be null, not both.
int swiglu_launch(float* out, uint16_t* out16, const float* gate, const float* up, int64_t n,
                  hipStream_t s) {
    if ((!out && !out16) || !gate || !up || n < 0) return FENCE_ERROR_INVALID_VALUE;
    if ((out && !aligned(out, 4)) || (out16 && !aligned(out16, 2)) || !aligned(gate, 4) || !aligned(up, 4))
        return FENCE_ERROR_INVALID_VALUE;
    if (n == 0) return FENCE_SUCCESS;
    const bool vec = (!out || aligned(out, 16)) && (!out16 || aligned(out16, 8)) && aligned(gate, 16) &&
                     aligned(up, 16);
    int64_t done = 0;
    if (vec) {
        const int64_t n4 = n / 4;
        // one launch per kMaxLaunchLanes lanes (each lane kSwigluUnroll float4s)
        constexpr int64_t kChunk4 = kMaxLaunchLanes * kSwigluUnroll;
        for (int64_t c0 = 0; c0 < n4; c0 += kChunk4) {
            const int64_t m4 = n4 - c0 < kChunk4 ? n4 - c0 : kChunk4;
            const unsigned grid = grid_1d(m4, kSwigluThreads * kSwigluUnroll);
            float* o = out ? out + 4 * c0 : nullptr;
            uint16_t* o16 = out16 ? out16 + 4 * c0 : nullptr;
            const float* g = gate + 4 * c0;
            const float* u = up + 4 * c0;
            int st;
            if (out && !out16) st = launch_swiglu_vec<true, false>(grid, s, o, o16, g, u, m4);
            else if (!out) st = launch_swiglu_vec<false, true>(grid, s, o, o16, g, u, m4);
            else st = launch_swiglu_vec<true, true>(grid, s, o, o16, g, u, m4);
            if (st) return st;
        }
        done = n4 * 4;
    }
    if (done < n) {
        const unsigned grid = grid_1d(n - done, kSwigluThreads, 65536);
        return launch(swiglu_scalar_kernel, dim3(grid), dim3(kSwigluThreads), 0, s, out, out16, gate, up,
                      done, n);
    }
    return FENCE_SUCCESS;
}

}  // namespace
}  // namespace fence

extern "C" int fence_swiglu(float* out, const float* gate, const float* up, int64_t n,
                            hipStream_t stream) {
    if (!out) return FENCE_ERROR_INVALID_VALUE;
    return fence::swiglu_launch(out, nullptr, gate, up, n, stream);
}

extern "C" int fence_silu_elementwise_mul(float* out, const float* gate, const float* up, int n,
                                          hipStream_t stream) {
    if (!out || n < 0) return FENCE_ERROR_INVALID_VALUE;
    return fence::swiglu_launch(out, nullptr, gate, up, n, stream);
}

extern "C" int fence_swiglu_f16(void* out_f16, float* out, const float* gate, const float* up,
                                int64_t n, hipStream_t stream) {
    if (!out_f16) return FENCE_ERROR_INVALID_VALUE;
    return fence::swiglu_launch(out, static_cast<uint16_t*>(out_f16), gate, up, n, stream);
}
