// common.hpp -- shared device and host helpers for the gfx950 kernels.
//
// Wave64 reductions use DPP lane permutes inside 16-lane rows and
// v_readlane across rows, so a row reduction finishes without LDS traffic
// and every lane of a group ends with the bitwise-identical value.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <tuple>
#include <type_traits>
#include <utility>

#include "fence/ops.h"

namespace fence {

constexpr int kWave = 64;

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ memory

template <bool NT>
__device__ __forceinline__ f4 ld4(const float* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const f4*>(p));
    else return *reinterpret_cast<const f4*>(p);
}

template <bool NT>
__device__ __forceinline__ void st4(float* p, f4 v) {
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<f4*>(p));
    else *reinterpret_cast<f4*>(p) = v;
}

typedef _Float16 h4 __attribute__((ext_vector_type(4)));

// binary32 -> binary16 by the hardware conversion (v_cvt_f16_f32): round to
// nearest even, overflow to inf, binary16 subnormals kept (the default MODE).
// The empty asm makes v an fp32 value first: otherwise the compiler may fold
// the multiply that produced it and the conversion into one v_fma_mixlo_f16,
// which rounds the exact product to binary16 once -- not what the reference's
// chain does (an fp32 result in memory, then f32_to_f16), and different
// whenever the fp32 rounding lands on a binary16 tie.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    asm volatile("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// Four binary16 values rounded from a float4, one 64-bit store (p 8-byte
// aligned); fp32 first, as above.
template <bool NT>
__device__ __forceinline__ void st_h4(uint16_t* p, f4 v) {
    asm volatile("" : "+v"(v));
    const h4 h = __builtin_convertvector(v, h4);
    if constexpr (NT) __builtin_nontemporal_store(h, reinterpret_cast<h4*>(p));
    else *reinterpret_cast<h4*>(p) = h;
}

// e^x as 2^(x log2 e) on the hardware's base-2 exponential (v_exp_f32), one
// multiply and one transcendental instead of the device library's
// extended-precision range reduction.  The rounding of x log2 e costs a
// relative error of about ln2 |x log2 e| 2^-24 (under 1e-6 for |x| < 16), plus
// the instruction's own ~1 ulp; +-inf and NaN map to 0 / inf / NaN as e^x does.
__device__ __forceinline__ float exp_hw(float x) {
    return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f);
}

// silu(g) * u of silu_elementwise_mul, src/kernels/ops.cuh:183-202,
// (g / (1 + e^-g)) * up, with e^-g from exp_hw and the quotient as g times the
// hardware reciprocal of 1 + e^-g (v_rcp_f32, ~1 ulp): about 5 VALU
// operations per element against ~25 for expf and an IEEE division, which
// matters in a 2-read/1-write stream.  Within ~1e-6 relative of the formula for
// |g| < 16; g = -inf gives NaN and large negative g gives -0, as the formula
// does.  Every kernel that produces SwiGLU activations uses this one
// expression, so fused and unfused paths round identically.
__device__ __forceinline__ float silu_mul(float g, float u) {
    return (g * __builtin_amdgcn_rcpf(1.0f + exp_hw(-g))) * u;
}

// Pairwise (a0^2 + a1^2) + (a2^2 + a3^2), four products and three sums with
// no fused multiply-add: the same rounding wherever it is inlined, so kernels
// that sum a row's squares in the same order agree bit for bit.
__device__ __forceinline__ float dot4(f4 a) {
#pragma clang fp contract(off)
    return (a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w);
}

// ------------------------------------------------------------- reductions

struct OpAdd {
    __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
    __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// DPP controls (GFX9 encoding).
enum : int {
    kDppQuadXor1 = 0xB1,   // quad_perm [1,0,3,2]
    kDppQuadXor2 = 0x4E,   // quad_perm [2,3,0,1]
    kDppHalfMirror = 0x141,// lane i <- lane 7-i within 8
    kDppMirror = 0x140,    // lane i <- lane 15-i within 16
    kDppRowNewBcast0 = 0x150,  // + n: every lane <- lane n of its 16-lane row (row_newbcast:n)
};

// Every control used here permutes lanes inside a 16-lane row, so with all
// lanes active no source is out of range and bound_ctrl never applies; setting
// it lets the compiler fold the move into the consuming VALU op (v_add_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// xor-16 exchange inside 32-lane halves (ds_swizzle bit mode: and=0x1F, xor=0x10)
__device__ __forceinline__ float swz_xor16(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}

// f(std::integral_constant<int, i>) for i = I .. N - 1: a loop whose index is
// a compile-time constant in the body (DPP controls must be).
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

__device__ __forceinline__ float readlane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Reduction over aligned groups of G lanes (G in {8,16,32}); every lane of a
// group receives the group result.  All 64 lanes must be active.
template <int G, class Op>
__device__ __forceinline__ float group_reduce(float v, Op op) {
    static_assert(G == 8 || G == 16 || G == 32, "group size");
    v = op(v, dpp<kDppQuadXor1>(v));
    v = op(v, dpp<kDppQuadXor2>(v));
    v = op(v, dpp<kDppHalfMirror>(v));
    if constexpr (G >= 16) v = op(v, dpp<kDppMirror>(v));
    if constexpr (G >= 32) v = op(v, swz_xor16(v));
    return v;
}

// Full-wave reduction; the result is wave-uniform.  All 64 lanes must be active.
template <class Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
    v = group_reduce<16>(v, op);
    return op(op(readlane(v, 0), readlane(v, 16)), op(readlane(v, 32), readlane(v, 48)));
}

// Workgroup reduction for blockDim.x = NWAVES * 64.  `scratch` holds NWAVES
// floats of LDS.  Ends with a barrier-protected read, so the result is
// uniform across the workgroup; callers may reuse `scratch` only after
// another __syncthreads().
template <int NWAVES, class Op>
__device__ __forceinline__ float block_reduce(float v, Op op, float* scratch) {
    v = wave_reduce(v, op);
    if constexpr (NWAVES == 1) {
        return v;
    } else {
        const int wave = threadIdx.x / kWave;
        if ((threadIdx.x % kWave) == 0) scratch[wave] = v;
        __syncthreads();
        float r = scratch[0];
#pragma unroll
        for (int i = 1; i < NWAVES; ++i) r = op(r, scratch[i]);
        return r;
    }
}

// Runtime wave count version (blockDim.x multiple of 64, at most 16 waves).
template <class Op>
__device__ __forceinline__ float block_reduce_dyn(float v, Op op, float* scratch) {
    v = wave_reduce(v, op);
    const int nwaves = blockDim.x / kWave;
    if (nwaves == 1) return v;
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x % kWave) == 0) scratch[wave] = v;
    __syncthreads();
    float r = scratch[0];
    for (int i = 1; i < nwaves; ++i) r = op(r, scratch[i]);
    return r;
}

// ------------------------------------------------------------------- host

inline bool aligned(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

inline int hip_status(hipError_t e) {
    return e == hipSuccess ? FENCE_SUCCESS : FENCE_ERROR_HIP_BASE + static_cast<int>(e);
}

// One-shot start/stop events for the next launch on this host thread
// (fence_time_next_launch).
// Events for the next `count` launches on this thread: `start` at the first
// one's kernel start, `stop` at the last one's kernel end.
struct TimingHook {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
    int count = 0;
};
inline TimingHook& timing_hook() {
    thread_local TimingHook hook;
    return hook;
}

template <class... KArgs, class Tuple, size_t... I>
inline int launch_impl(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t shmem,
                       hipStream_t stream, Tuple& args, std::index_sequence<I...>) {
    void* ptrs[] = {static_cast<void*>(&std::get<I>(args))..., nullptr};
    TimingHook& hook = timing_hook();
    if (hook.count > 0) {
        const hipEvent_t a = hook.start;
        const hipEvent_t b = hook.count == 1 ? hook.stop : nullptr;
        hook.start = nullptr;
        if (--hook.count == 0) hook = TimingHook{};
        return hip_status(hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block,
                                             ptrs, shmem, stream, a, b, 0));
    }
    return hip_status(hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block,
                                      ptrs, shmem, stream));
}

// Launch `kernel` and return the status of this launch (not of earlier calls).
template <class... KArgs, class... Args>
inline int launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t shmem,
                  hipStream_t stream, Args&&... args) {
    static_assert(sizeof...(KArgs) == sizeof...(Args), "kernel argument count");
    std::tuple<KArgs...> packed(std::forward<Args>(args)...);
    return launch_impl(kernel, grid, block, shmem, stream, packed,
                       std::index_sequence_for<KArgs...>{});
}

// Threads per row (a multiple of 64, at most 1024) and items per lane for
// `rows` rows of `items` vector items each, aiming at `target` items per lane.
// Measured on MI355X: a 2048-float softmax row runs at 82% of HBM peak with
// 256 lanes x 2 float4 but 62% with 512 lanes x 1 -- fewer, fuller lanes per
// row keep more rows in flight per CU -- while a grid too small to fill the
// GPU (512 tokens of 40 heads) does better with wider rows.  So the target is
// halved while the grid would hold fewer waves than the GPU runs at once.
// Returns false if a row needs more than max_per_lane items per lane.
constexpr int64_t kGpuWaves = 256 * 32;  // 256 CUs x 32 resident waves

inline bool plan_row(int64_t rows, int64_t items, int target, int max_per_lane, unsigned* threads,
                     int* per_lane) {
    while (target > 1 && rows * ((items + 64 * target - 1) / (64 * target)) < kGpuWaves) target /= 2;
    int64_t t = (items + target - 1) / target;
    t = (t + 63) / 64 * 64;
    if (t < 64) t = 64;
    if (t > 1024) t = 1024;
    const int64_t pl = (items + t - 1) / t;
    if (pl > max_per_lane) return false;
    *threads = static_cast<unsigned>(t);
    *per_lane = static_cast<int>(pl);
    return true;
}

// Reduction over the WPR consecutive waves that share one row (WPR waves per
// row, several rows per workgroup).  `scratch` holds one float per wave of the
// workgroup; callers must barrier before reusing it.
template <int WPR, class Op>
__device__ __forceinline__ float row_reduce(float v, Op op, float* scratch) {
    v = wave_reduce(v, op);
    if constexpr (WPR == 1) {
        return v;
    } else {
        const int wave = threadIdx.x / kWave;
        if ((threadIdx.x % kWave) == 0) scratch[wave] = v;
        __syncthreads();
        const int first = (wave / WPR) * WPR;
        float r = scratch[first];
#pragma unroll
        for (int i = 1; i < WPR; ++i) r = op(r, scratch[first + i]);
        return r;
    }
}

// The vector row RMSNorm's launch shape (rms_norm.hip): threads per row and
// float4s per lane for rows of n floats.  Its sum of squares is ordered by
// this shape, so a kernel that normalises a row itself (the Q6_K GEMV's
// prologue) takes the shape from here to sum in the same order.
#ifndef FENCE_RMS_VPT
#define FENCE_RMS_VPT 2
#endif
inline bool rms_row_plan(int64_t rows, int n, unsigned* threads, int* vpt) {
    return plan_row(rows, n / 4, FENCE_RMS_VPT, 8, threads, vpt);
}

// One row: x16 = binary16(rms_norm(hid + res) * w), hid_out = hid + res (res
// may be null: the row is hid and hid_out is not written).  rms_norm.hip.
int residual_rms_f16_launch(float* hid_out, uint16_t* x16, const float* hid, const float* res, const float* w,
                            int n, float eps, hipStream_t s);

// Lanes one launch of a one-pass kernel may cover.  A dispatch's grid size in
// lanes is a 32-bit field, so arrays beyond this take several launches.
constexpr int64_t kMaxLaunchLanes = int64_t(1) << 30;

inline unsigned grid_1d(int64_t units, int64_t per_block, int64_t cap = 1 << 30) {
    int64_t g = (units + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return static_cast<unsigned>(g);
}

}  // namespace fence
