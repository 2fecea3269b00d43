// rms_norm.hip -- row RMSNorm on gfx950, alone or as the layer-boundary
// epilogue (residual add -> RMSNorm -> binary16).
//
// Follows rms_norm, src/kernels/ops.cuh:17-51:
//   r = rsqrt(sum(x^2) / n + eps);  out[i] = (w[i] * x[i]) * r.
// The epilogue form composes what src/model/qwen3.cu:310-325 runs as three
// kernels and a copy between two GEMVs: residual_add (ops.cuh:256-270,
// hidden += residual, the sum also being the next sub-block's residual),
// rms_norm, and f32_to_f16 (ops.cuh:448-462, round to nearest even) of the
// normalised row for the next GEMV's input.
// The reference runs one 1024-thread block and reads x twice.  Here one
// workgroup owns one row; the row (and its residual) is read once with
// 128-bit loads -- about two float4 per lane, all issued before any is
// consumed -- and kept in VGPRs, the sum of squares is reduced with DPP
// inside each wave and one LDS exchange across waves, and the outputs are
// written from the registers.  out may equal x, and hidden may equal x:
// every element is read before the reduction's barrier and written after it,
// by the lane that read it.
#include <type_traits>

#include "common.hpp"

namespace fence {
namespace {

constexpr int kMaxWaves = 16;

// Row outputs: OUT32 writes the fp32 normalised row to `out`, OUT16 its
// binary16 rounding to `out16`; RES adds `res` to the row first and writes
// the sum to `hid`.
template <int MAXV, bool RES, bool OUT32, bool OUT16>
__global__ __launch_bounds__(1024) void rms_rows_vec_kernel(
    float* out, uint16_t* out16, float* hid, const float* x, const float* res, const float* w,
    int64_t rows, int n, int vpt, float eps) {
    __shared__ float red[kMaxWaves];
    const int T = blockDim.x;
    const int n4 = n >> 2;
    f4 wv[MAXV];  // the weights: the same for every row, loaded once
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
        const int f = threadIdx.x + j * T;
        wv[j] = (j < vpt && f < n4) ? ld4<false>(w + 4 * f) : f4(0.0f);
    }
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + r * n;
        f4 v[MAXV], rv[MAXV];
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {  // all loads of the row first
            const int f = threadIdx.x + j * T;
            v[j] = f4(0.0f);
            rv[j] = f4(0.0f);
            if (j < vpt && f < n4) {
                v[j] = ld4<true>(xr + 4 * f);
                if constexpr (RES) rv[j] = ld4<true>(res + r * n + 4 * f);
            }
        }
        if constexpr (RES) {
#pragma unroll
            for (int j = 0; j < MAXV; ++j) {
                const int f = threadIdx.x + j * T;
                v[j] = v[j] + rv[j];
                if (j < vpt && f < n4) st4<true>(hid + r * n + 4 * f, v[j]);
            }
        }
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXV; ++j) ss += dot4(v[j]);
        const float tot = block_reduce_dyn(ss, OpAdd(), red);
        const float rs = rsqrtf(tot / static_cast<float>(n) + eps);
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int f = threadIdx.x + j * T;
            if (j < vpt && f < n4) {
                const f4 o = (wv[j] * v[j]) * rs;
                if constexpr (OUT32) st4<true>(out + r * n + 4 * f, o);
                if constexpr (OUT16) st_h4<true>(out16 + r * n + 4 * f, o);
            }
        }
        __syncthreads();  // red[] is rewritten by the next row
    }
}

// Any n and alignment: read the row twice with scalar accesses.
__global__ __launch_bounds__(256) void rms_rows_scalar_kernel(
    float* out, uint16_t* out16, float* hid, const float* x, const float* res, const float* w,
    int64_t rows, int n, float eps) {
    __shared__ float red[4];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + r * n;
        float ss = 0.0f;
        for (int i = threadIdx.x; i < n; i += 256) {
            float v = xr[i];
            if (res) {
                v += res[r * n + i];
                hid[r * n + i] = v;
            }
            ss += v * v;
        }
        // the sums written above are re-read below by the lanes that wrote them
        const float tot = block_reduce<4>(ss, OpAdd(), red);
        const float rs = rsqrtf(tot / static_cast<float>(n) + eps);
        const float* vr = res ? hid + r * n : xr;
        for (int i = threadIdx.x; i < n; i += 256) {
            const float o = (w[i] * vr[i]) * rs;
            if (out) out[r * n + i] = o;
            if (out16) out16[r * n + i] = f32_to_f16_bits(o);
        }
        __syncthreads();
    }
}

template <bool RES, bool OUT32, bool OUT16>
int launch_vec(unsigned grid, unsigned threads, int vpt, hipStream_t s, float* out, uint16_t* out16,
               float* hid, const float* x, const float* res, const float* w, int64_t rows, int n,
               float eps) {
    if (vpt <= 2)
        return launch(rms_rows_vec_kernel<2, RES, OUT32, OUT16>, dim3(grid), dim3(threads), 0, s, out,
                      out16, hid, x, res, w, rows, n, vpt, eps);
    return launch(rms_rows_vec_kernel<8, RES, OUT32, OUT16>, dim3(grid), dim3(threads), 0, s, out, out16,
                  hid, x, res, w, rows, n, vpt, eps);
}

// out / out16: either may be null (not both); res null = no residual add.
int rms_rows_launch(float* out, uint16_t* out16, float* hid, const float* x, const float* res,
                    const float* w, int64_t rows, int n, float eps, hipStream_t s) {
    if ((!out && !out16) || !x || !w || (res && !hid) || rows < 0 || n <= 0)
        return FENCE_ERROR_INVALID_VALUE;
    if (res && out == hid) return FENCE_ERROR_INVALID_VALUE;  // would overwrite the sum
    if ((out && !aligned(out, 4)) || !aligned(x, 4) || !aligned(w, 4) || (res && !aligned(res, 4)) ||
        (hid && !aligned(hid, 4)) || (out16 && !aligned(out16, 2)))
        return FENCE_ERROR_INVALID_VALUE;
    if (rows == 0) return FENCE_SUCCESS;
    const unsigned grid = grid_1d(rows, 1, 1 << 20);
    const bool vec = (n % 4 == 0) && (!out || aligned(out, 16)) && aligned(x, 16) && aligned(w, 16) &&
                     (!res || (aligned(res, 16) && aligned(hid, 16))) && (!out16 || aligned(out16, 8));
    unsigned threads = 0;
    int vpt = 0;
    if (vec && rms_row_plan(rows, n, &threads, &vpt)) {
        const auto go = [&](auto res_c, auto o32_c, auto o16_c) {
            return launch_vec<decltype(res_c)::value, decltype(o32_c)::value, decltype(o16_c)::value>(
                grid, threads, vpt, s, out, out16, hid, x, res, w, rows, n, eps);
        };
        using T = std::true_type;
        using F = std::false_type;
        if (!res && out && !out16) return go(F{}, T{}, F{});
        if (!res && !out && out16) return go(F{}, F{}, T{});
        if (!res && out && out16) return go(F{}, T{}, T{});
        if (res && out && !out16) return go(T{}, T{}, F{});
        if (res && !out && out16) return go(T{}, F{}, T{});
        return go(T{}, T{}, T{});
    }
    return launch(rms_rows_scalar_kernel, dim3(grid), dim3(256), 0, s, out, out16, hid, x, res, w, rows,
                  n, eps);
}

}  // namespace

int residual_rms_f16_launch(float* hid_out, uint16_t* x16, const float* hid, const float* res, const float* w,
                            int n, float eps, hipStream_t s) {
    if (!x16) return FENCE_ERROR_INVALID_VALUE;
    return rms_rows_launch(nullptr, x16, hid_out, hid, res, w, 1, n, eps, s);
}

int rms_norm_rows_launch(float* out, const float* x, const float* w, int64_t rows, int n,
                         float eps, hipStream_t s) {
    if (!out) return FENCE_ERROR_INVALID_VALUE;
    return rms_rows_launch(out, nullptr, nullptr, x, nullptr, w, rows, n, eps, s);
}

}  // namespace fence

extern "C" int fence_rms_norm(float* out, const float* x, const float* w, int n, float eps,
                              hipStream_t stream) {
    return fence::rms_norm_rows_launch(out, x, w, 1, n, eps, stream);
}

extern "C" int fence_rms_norm_inplace(float* x, const float* w, int n, float eps,
                                      hipStream_t stream) {
    return fence::rms_norm_rows_launch(x, x, w, 1, n, eps, stream);
}

extern "C" int fence_rms_norm_rows(float* out, const float* x, const float* w, int64_t rows, int n,
                                   float eps, hipStream_t stream) {
    return fence::rms_norm_rows_launch(out, x, w, rows, n, eps, stream);
}

extern "C" int fence_residual_rms_norm_f16(float* hidden, const float* residual, const float* w,
                                           float* normed, void* out_f16, int64_t rows, int n,
                                           float eps, hipStream_t stream) {
    if (!hidden) return FENCE_ERROR_INVALID_VALUE;
    return fence::rms_rows_launch(normed, static_cast<uint16_t*>(out_f16), hidden, hidden, residual, w,
                                  rows, n, eps, stream);
}
