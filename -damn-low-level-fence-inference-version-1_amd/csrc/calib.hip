// calib.hip -- plain float4 streams for measuring the attainable HBM rate on
// gfx950.  No reference counterpart: a benchmark times these next to the
// ops, so each op's bandwidth can be read against what a stream of the same
// read/write mix reaches on the same device, rather than only against the
// 8 TB/s datasheet peak.
//
//   b != null: out[i] = a[i] + b[i]   (2 reads, 1 write: SwiGLU's traffic)
//   b == null: out[i] = a[i]          (1 read, 1 write; out == a is the
//                                      in-place form, RoPE's traffic)
//   a == null: out[i] = 0             (1 write: the masked half of the
//                                      causal softmax's output)
//   fence_calib_read: sums[w] = the sum of what wave w read (1 read: a
//                     GEMV's weight stream; one float written per wave)
//
// Each lane moves VPT float4s of every stream with non-temporal 128-bit loads
// and stores (the elementwise kernels' memory access), THREADS lanes per
// workgroup, one workgroup per THREADS * VPT float4s.  The launch shape is an
// argument so the caller can sweep it and keep the fastest.
#include "common.hpp"

namespace fence {
namespace {

// READS: streams read (0: out = 0, 1: out = a, 2: out = a + b).
template <int THREADS, int VPT, int READS>
__global__ __launch_bounds__(THREADS) void calib_stream_kernel(float* out, const float* a, const float* b,
                                                               int64_t n4) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * (THREADS * VPT) + threadIdx.x;
    f4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t i = base + static_cast<int64_t>(j) * THREADS;
        v[j] = f4(0.0f);
        if (READS > 0 && i < n4) {
            v[j] = ld4<true>(a + 4 * i);
            if constexpr (READS == 2) v[j] += ld4<true>(b + 4 * i);
        }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t i = base + static_cast<int64_t>(j) * THREADS;
        if (i < n4) st4<true>(out + 4 * i, v[j]);
    }
}

// Read-only: each lane adds the components of its VPT float4s, and lane 0
// of each wave stores the wave's sum, so no load can be dropped and the
// writes are 4 bytes per 1,024 * VPT read.
template <int THREADS, int VPT>
__global__ __launch_bounds__(THREADS) void calib_read_kernel(float* sums, const float* a, int64_t n4) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * (THREADS * VPT) + threadIdx.x;
    f4 v[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int64_t i = base + static_cast<int64_t>(j) * THREADS;
        v[j] = i < n4 ? ld4<true>(a + 4 * i) : f4(0.0f);
    }
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) acc += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    acc = wave_reduce(acc, OpAdd{});
    if ((threadIdx.x & (kWave - 1)) == 0)
        sums[static_cast<int64_t>(blockIdx.x) * (THREADS / kWave) + threadIdx.x / kWave] = acc;
}

template <int THREADS, int VPT>
int calib_launch(float* out, const float* a, const float* b, int64_t n4, hipStream_t s) {
    const unsigned grid = grid_1d(n4, THREADS * VPT);
    if (!a) return launch(calib_stream_kernel<THREADS, VPT, 0>, dim3(grid), dim3(THREADS), 0, s, out, a, b, n4);
    if (b) return launch(calib_stream_kernel<THREADS, VPT, 2>, dim3(grid), dim3(THREADS), 0, s, out, a, b, n4);
    return launch(calib_stream_kernel<THREADS, VPT, 1>, dim3(grid), dim3(THREADS), 0, s, out, a, b, n4);
}

template <int THREADS>
int calib_vpt(int vpt, float* out, const float* a, const float* b, int64_t n4, hipStream_t s) {
    switch (vpt) {
        case 1: return calib_launch<THREADS, 1>(out, a, b, n4, s);
        case 2: return calib_launch<THREADS, 2>(out, a, b, n4, s);
        case 4: return calib_launch<THREADS, 4>(out, a, b, n4, s);
        default: return FENCE_ERROR_INVALID_VALUE;
    }
}

template <int THREADS>
int calib_read_vpt(int vpt, float* sums, const float* a, int64_t n4, hipStream_t s) {
    switch (vpt) {
        case 1: return launch(calib_read_kernel<THREADS, 1>, dim3(grid_1d(n4, THREADS)), dim3(THREADS), 0, s, sums, a, n4);
        case 2: return launch(calib_read_kernel<THREADS, 2>, dim3(grid_1d(n4, THREADS * 2)), dim3(THREADS), 0, s, sums, a, n4);
        case 4: return launch(calib_read_kernel<THREADS, 4>, dim3(grid_1d(n4, THREADS * 4)), dim3(THREADS), 0, s, sums, a, n4);
        default: return FENCE_ERROR_INVALID_VALUE;
    }
}

}  // namespace
}  // namespace fence

extern "C" int fence_calib_stream(float* out, const float* a, const float* b, int64_t n, int threads, int vpt,
                                  hipStream_t stream) {
    using namespace fence;
    if (!out || (!a && b) || n < 0 || n % 4 != 0) return FENCE_ERROR_INVALID_VALUE;
    if (!aligned(out, 16) || (a && !aligned(a, 16)) || (b && !aligned(b, 16))) return FENCE_ERROR_INVALID_VALUE;
    const int64_t n4 = n / 4;
    // one launch's grid must stay within a dispatch's 32-bit lane count
    if (n4 > kMaxLaunchLanes) return FENCE_ERROR_INVALID_VALUE;
    if (n4 == 0) return FENCE_SUCCESS;
    switch (threads) {
        case 64: return calib_vpt<64>(vpt, out, a, b, n4, stream);
        case 256: return calib_vpt<256>(vpt, out, a, b, n4, stream);
        default: return FENCE_ERROR_INVALID_VALUE;
    }
}

extern "C" int fence_calib_read(float* sums, const float* a, int64_t n, int threads, int vpt, hipStream_t stream) {
    using namespace fence;
    if (!sums || !a || n < 0 || n % 4 != 0 || !aligned(a, 16)) return FENCE_ERROR_INVALID_VALUE;
    const int64_t n4 = n / 4;
    if (n4 > kMaxLaunchLanes) return FENCE_ERROR_INVALID_VALUE;
    if (n4 == 0) return FENCE_SUCCESS;
    switch (threads) {
        case 64: return calib_read_vpt<64>(vpt, sums, a, n4, stream);
        case 256: return calib_read_vpt<256>(vpt, sums, a, n4, stream);
        default: return FENCE_ERROR_INVALID_VALUE;
    }
}
