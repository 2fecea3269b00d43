// convert.hip -- the elementwise epilogue ops of a decode step on gfx950:
// residual add and the binary32 <-> binary16 conversions.
//
// Follows residual_add (src/kernels/ops.cuh:256-270, x[i] += residual[i]),
// f32_to_f16 (:448-462) and float_to_half (:274-289), both
// out[i] = __float2half(in[i]) with round to nearest even, and half_to_float
// (:293-308, exact).  Streaming kernels: one float4 (or four binary16) per
// lane per stream, non-temporal 128-bit / 64-bit accesses; a scalar form
// takes unaligned pointers and the n % 4 tail.
#include "common.hpp"

namespace fence {
namespace {

constexpr int kThreads = 256;

enum class Op { kResidualAdd, kToF16, kToF32 };

template <Op OP>
__global__ __launch_bounds__(kThreads) void convert_vec_kernel(void* dst, const void* src, int64_t n4) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n4) return;
    if constexpr (OP == Op::kResidualAdd) {
        float* x = static_cast<float*>(dst);
        const f4 a = ld4<true>(x + 4 * i);
        const f4 b = ld4<true>(static_cast<const float*>(src) + 4 * i);
        st4<true>(x + 4 * i, a + b);
    } else if constexpr (OP == Op::kToF16) {
        st_h4<true>(static_cast<uint16_t*>(dst) + 4 * i, ld4<true>(static_cast<const float*>(src) + 4 * i));
    } else {
        const h4 h = __builtin_nontemporal_load(reinterpret_cast<const h4*>(src) + i);
        st4<true>(static_cast<float*>(dst) + 4 * i, __builtin_convertvector(h, f4));
    }
}

template <Op OP>
__global__ __launch_bounds__(kThreads) void convert_scalar_kernel(void* dst, const void* src, int64_t begin,
                                                                  int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    for (int64_t i = begin + static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n; i += stride) {
        if constexpr (OP == Op::kResidualAdd)
            static_cast<float*>(dst)[i] += static_cast<const float*>(src)[i];
        else if constexpr (OP == Op::kToF16)
            static_cast<uint16_t*>(dst)[i] = f32_to_f16_bits(static_cast<const float*>(src)[i]);
        else
            static_cast<float*>(dst)[i] =
                static_cast<float>(__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(src)[i]));
    }
}

template <Op OP>
int convert_launch(void* dst, const void* src, int64_t n, hipStream_t s) {
    constexpr size_t dst_size = OP == Op::kToF16 ? 2 : 4;
    constexpr size_t src_size = OP == Op::kToF32 ? 2 : 4;
    if (!dst || !src || n < 0) return FENCE_ERROR_INVALID_VALUE;
    if (!aligned(dst, dst_size) || !aligned(src, src_size)) return FENCE_ERROR_INVALID_VALUE;
    if (n == 0) return FENCE_SUCCESS;
    int64_t done = 0;
    if (aligned(dst, 4 * dst_size) && aligned(src, 4 * src_size)) {
        const int64_t n4 = n / 4;
        for (int64_t c0 = 0; c0 < n4; c0 += kMaxLaunchLanes) {  // one launch per kMaxLaunchLanes float4s
            const int64_t m4 = n4 - c0 < kMaxLaunchLanes ? n4 - c0 : kMaxLaunchLanes;
            void* d = static_cast<uint8_t*>(dst) + 4 * dst_size * c0;
            const void* sp = static_cast<const uint8_t*>(src) + 4 * src_size * c0;
            if (int st = launch(convert_vec_kernel<OP>, dim3(grid_1d(m4, kThreads)), dim3(kThreads), 0, s, d, sp, m4))
                return st;
        }
        done = n4 * 4;
    }
    if (done < n)
        return launch(convert_scalar_kernel<OP>, dim3(grid_1d(n - done, kThreads, 65536)), dim3(kThreads), 0, s,
                      dst, src, done, n);
    return FENCE_SUCCESS;
}

}  // namespace
}  // namespace fence

extern "C" int fence_residual_add(float* x, const float* residual, int n, hipStream_t stream) {
    return fence::convert_launch<fence::Op::kResidualAdd>(x, residual, n, stream);
}

extern "C" int fence_f32_to_f16(void* out, const float* in, int n, hipStream_t stream) {
    return fence::convert_launch<fence::Op::kToF16>(out, in, n, stream);
}

extern "C" int fence_f16_to_f32(float* out, const void* in, int n, hipStream_t stream) {
    return fence::convert_launch<fence::Op::kToF32>(out, in, n, stream);
}
