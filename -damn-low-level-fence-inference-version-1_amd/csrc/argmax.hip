// argmax.hip -- greedy-sampling argmax over fp32 logits, on gfx950.
//
// Follows argmax_kernel / argmax, src/kernels/ops.cuh:467-505: one block of
// 256 threads; thread t scans x[t], x[t+256], ... keeping the first value
// strictly greater than its running maximum (initially -1e30f, index 0), then
// a shared-memory tree (s = 128, 64, .., 1) lets slot u take slot u+s only if
// that value is strictly greater.  The tree decides ties: level s pairs
// threads that differ in bit log2(s) and the lower slot keeps an equal value,
// so among the threads holding the maximum the one with the smallest 8-bit
// bit-reversal of t wins (bits compared from the lowest up), and within a
// thread the first index does.  Equal maxima at 1 and 256 give 256 (thread
// 0), at 1 and 2 give 2 (reversals 128 and 64).
//
// That whole rule is one total order, so here every element becomes a 64-bit
// key and any reduction order gives the reference's result:
//   key(i) = ord(x[i]) << 32 | ~(rev8(i mod 256) << 23 | i >> 8)
// for x[i] > -1e30f (NaN and values at or below -1e30 never qualify), key 0
// otherwise; ord() orders floats as integers with -0 and +0 equal.  The
// largest key names the result; key 0 (nothing qualifies) gives index 0, as
// in the reference.  Indices i < 2^31 keep i >> 8 within 23 bits.
//
// Within one thread the elements of one class (i mod 256) are visited in
// increasing index, because every stride below is a multiple of 256 floats;
// so a thread tracks the first strict maximum per class it visits and forms
// keys once, at the end.
#include "common.hpp"

#include <mutex>

namespace fence {
namespace {

constexpr float kArgmaxInit = -1e30f;   // the reference's initial maximum
constexpr int kArgmaxMaxParts = 1024;    // workgroups of the multi-workgroup form

__device__ __forceinline__ uint64_t argmax_key(float v, int i) {
    uint32_t b = __float_as_uint(v);
    if ((b << 1) == 0) b = 0;  // -0 ties with +0
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    const uint32_t pri = ((__brev(static_cast<uint32_t>(i) & 255u) >> 24) << 23) | (static_cast<uint32_t>(i) >> 8);
    return (static_cast<uint64_t>(ord) << 32) | static_cast<uint32_t>(~pri);
}

__device__ __forceinline__ int key_index(uint64_t key) {
    if (key == 0) return 0;
    const uint32_t pri = ~static_cast<uint32_t>(key);
    return static_cast<int>(((pri & 0x7FFFFFu) << 8) | (__brev(pri >> 23) >> 24));
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Largest key of the workgroup (blockDim.x = 64 * waves, waves <= 16); the
// result is valid in every lane of wave 0.
__device__ __forceinline__ uint64_t block_max_key(uint64_t k) {
    __shared__ uint64_t part[16];
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) k = umax64(k, shfl_xor64(k, m));
    const int waves = blockDim.x / kWave;
    if (waves == 1) return k;
    if ((threadIdx.x % kWave) == 0) part[threadIdx.x / kWave] = k;
    __syncthreads();
    k = (threadIdx.x < static_cast<unsigned>(waves)) ? part[threadIdx.x] : 0;
#pragma unroll
    for (int m = 8; m > 0; m >>= 1) k = umax64(k, shfl_xor64(k, m));
    return k;
}

// Workgroup b of gridDim.x scans float4 f = b*blockDim + t, then every
// gridDim.x*blockDim float4 after it (a multiple of 256 floats, so each of
// the four components stays in one class).  FINAL (one workgroup): writes
// the index; otherwise the workgroup's largest key to parts[b].
template <bool FINAL>
__global__ __launch_bounds__(1024) void argmax_kernel(int* __restrict__ result, uint64_t* __restrict__ parts,
                                                      const float* __restrict__ x, int n, int vec) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int stride = gridDim.x * blockDim.x;
    uint64_t key = 0;
    if (vec) {
        const int n4 = n >> 2;
        float bv[4] = {kArgmaxInit, kArgmaxInit, kArgmaxInit, kArgmaxInit};
        int bi[4] = {-1, -1, -1, -1};
        constexpr int kBatch = 4;  // float4 loads a lane has in flight
        for (int f0 = t; f0 < n4; f0 += stride * kBatch) {
            f4 v[kBatch];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const int f = f0 + stride * b;
                v[b] = ld4<true>(x + 4 * static_cast<int64_t>(f < n4 ? f : f0));  // clamped: inside x
            }
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {  // increasing index within each component
                const int f = f0 + stride * b;
                if (f < n4) {
                    if (v[b].x > bv[0]) bv[0] = v[b].x, bi[0] = 4 * f;
                    if (v[b].y > bv[1]) bv[1] = v[b].y, bi[1] = 4 * f + 1;
                    if (v[b].z > bv[2]) bv[2] = v[b].z, bi[2] = 4 * f + 2;
                    if (v[b].w > bv[3]) bv[3] = v[b].w, bi[3] = 4 * f + 3;
                }
            }
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (bi[c] >= 0) key = umax64(key, argmax_key(bv[c], bi[c]));
        // the last n % 4 elements, one per lane; in 64 bits, since 4 * n4 + t
        // passes INT_MAX when n is within one grid of it
        const int64_t tail = 4 * static_cast<int64_t>(n4) + t;
        if (tail < n) {
            const float v = x[tail];
            if (v > kArgmaxInit) key = umax64(key, argmax_key(v, static_cast<int>(tail)));
        }
    } else {
        float bv = kArgmaxInit;
        int bi = -1;
        for (int64_t i = t; i < n; i += stride)  // 64-bit: i + stride may pass INT_MAX
            if (x[i] > bv) bv = x[i], bi = static_cast<int>(i);
        if (bi >= 0) key = argmax_key(bv, bi);
    }
    key = block_max_key(key);
    if (threadIdx.x == 0) {
        if constexpr (FINAL) *result = key_index(key);
        else parts[blockIdx.x] = key;
    }
}

// One workgroup: the largest of `count` partial keys, as an index.
__global__ __launch_bounds__(256) void argmax_merge_kernel(int* __restrict__ result,
                                                           const uint64_t* __restrict__ parts, int count) {
    uint64_t key = 0;
    for (int i = threadIdx.x; i < count; i += blockDim.x) key = umax64(key, parts[i]);
    key = block_max_key(key);
    if (threadIdx.x == 0) *result = key_index(key);
}

}  // namespace

int argmax_launch(const float* x, int* result, int n, hipStream_t s) {
    if (!x || !result || n < 0 || !aligned(x, 4) || !aligned(result, 4)) return FENCE_ERROR_INVALID_VALUE;
    return launch(argmax_kernel<true>, dim3(1), dim3(1024), 0, s, result, static_cast<uint64_t*>(nullptr), x, n,
                  aligned(x, 16) ? 1 : 0);
}

// Workgroups for n elements: one float4 (or 4 scalars) per lane, at most
// kArgmaxMaxParts and at most `cap`.
int argmax_parts(int n, int64_t cap) {
    const int64_t lanes = (static_cast<int64_t>(n) + 3) / 4;
    int64_t g = (lanes + 255) / 256;
    if (g > kArgmaxMaxParts) g = kArgmaxMaxParts;
    if (g > cap) g = cap;
    return g < 1 ? 1 : static_cast<int>(g);
}

int argmax_parts_launch(const float* x, int* result, int n, uint64_t* parts, int count, hipStream_t s) {
    const int vec = aligned(x, 16) ? 1 : 0;
    int st = launch(argmax_kernel<false>, dim3(count), dim3(256), 0, s, static_cast<int*>(nullptr), parts, x, n,
                    vec);
    if (st != FENCE_SUCCESS) return st;
    return launch(argmax_merge_kernel, dim3(1), dim3(256), 0, s, result, static_cast<const uint64_t*>(parts),
                  count);
}

int argmax_ws_launch(const float* x, int* result, int n, void* workspace, int64_t workspace_bytes, hipStream_t s) {
    if (!x || !result || n < 0 || !aligned(x, 4) || !aligned(result, 4)) return FENCE_ERROR_INVALID_VALUE;
    if (!workspace || !aligned(workspace, 8) || workspace_bytes < static_cast<int64_t>(sizeof(uint64_t)))
        return FENCE_ERROR_INVALID_VALUE;
    const int count = argmax_parts(n, workspace_bytes / static_cast<int64_t>(sizeof(uint64_t)));
    return argmax_parts_launch(x, result, n, static_cast<uint64_t*>(workspace), count, s);
}

// ------------------------------------------------- allocation-free variant
//
// fence_argmax_noalloc keeps its partials in `scratch`, a file-scope device
// array: kArgmaxMaxParts keys, 8 KiB.  Every GPU the library runs on holds its
// own copy until the process ends, and every call on one GPU shares it, so
// calls that overlap on one GPU (two streams, two threads) race; calls
// ordered on one stream do not.  Nothing in it must start at zero: each call's
// first kernel writes every partial its second kernel reads.  In host code the
// array's name is not a device address, so the address each device gives for
// it (hipGetSymbolAddress, once per device, with that device current) is what
// the kernels get.

namespace {

static __device__ __align__(256) uint64_t scratch[kArgmaxMaxParts];

constexpr int kMaxDevices = 64;
uint64_t* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// This device's address of `scratch`, looked up on the device's first call.
// The stream must belong to the current device (the address is that
// device's); a stream of another device is rejected.
int scratch_ptr(hipStream_t s, uint64_t** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e);
    if (dev < 0 || dev >= kMaxDevices) return FENCE_ERROR_INVALID_VALUE;
    if (s) {
        int sdev = -1;
        e = hipStreamGetDevice(s, &sdev);
        if (e != hipSuccess) return hip_status(e);
        if (sdev != dev) return FENCE_ERROR_INVALID_VALUE;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e);
        if (!p) return FENCE_ERROR_INVALID_VALUE;
        g_scratch_ptr[dev] = static_cast<uint64_t*>(p);
    }
    *out = g_scratch_ptr[dev];
    return FENCE_SUCCESS;
}

}  // namespace

int argmax_noalloc_launch(const float* x, int* result, int n, hipStream_t s) {
    if (!x || !result || n < 0 || !aligned(x, 4) || !aligned(result, 4)) return FENCE_ERROR_INVALID_VALUE;
    uint64_t* parts = nullptr;
    const int st = scratch_ptr(s, &parts);
    if (st != FENCE_SUCCESS) return st;
    // every n fits: the grid is capped at kArgmaxMaxParts workgroups
    return argmax_parts_launch(x, result, n, parts, argmax_parts(n, kArgmaxMaxParts), s);
}

}  // namespace fence

extern "C" int fence_argmax(const float* x, int* result, int n, hipStream_t stream) {
    return fence::argmax_launch(x, result, n, stream);
}

extern "C" int fence_argmax_ws(const float* x, int* result, int n, void* workspace, int64_t workspace_bytes,
                               hipStream_t stream) {
    return fence::argmax_ws_launch(x, result, n, workspace, workspace_bytes, stream);
}

extern "C" int fence_argmax_noalloc(const float* x, int* result, int n, hipStream_t stream) {
    return fence::argmax_noalloc_launch(x, result, n, stream);
}
