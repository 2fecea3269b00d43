// rms_norm.hip -- row RMSNorm on gfx950.
//
// Follows rms_norm, src/kernels/ops.cuh:17-51:
//   r = rsqrt(sum(x^2) / n + eps);  out[i] = (w[i] * x[i]) * r.
// The reference runs one 1024-thread block and reads x twice.  Here one
// workgroup owns one row; the row is read once with 128-bit loads -- about
// two float4 per lane, all issued before any is consumed -- and kept in
// VGPRs, the sum of squares is reduced with DPP inside each wave and one LDS
// exchange across waves, and the normalised row is written from the
// registers.  out may equal x: every element is read before the reduction's
// barrier and written after it.
#include "common.hpp"

#ifndef FENCE_RMS_VPT
#define FENCE_RMS_VPT 2
#endif

namespace fence {
namespace {

constexpr int kMaxWaves = 16;

template <int MAXV>
__global__ __launch_bounds__(1024) void rms_rows_vec_kernel(
    float* out, const float* x, const float* w, int64_t rows, int n, int vpt, float eps) {
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
        float* orow = out + r * n;
        f4 v[MAXV];
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {  // all loads of the row first
            const int f = threadIdx.x + j * T;
            v[j] = f4(0.0f);
            if (j < vpt && f < n4) v[j] = ld4<true>(xr + 4 * f);
        }
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXV; ++j) ss += dot4(v[j]);
        const float tot = block_reduce_dyn(ss, OpAdd(), red);
        const float rs = rsqrtf(tot / static_cast<float>(n) + eps);
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int f = threadIdx.x + j * T;
            if (j < vpt && f < n4) st4<true>(orow + 4 * f, (wv[j] * v[j]) * rs);
        }
        __syncthreads();  // red[] is rewritten by the next row
    }
}

// Any n and alignment: read the row twice with scalar accesses.
__global__ __launch_bounds__(256) void rms_rows_scalar_kernel(
    float* out, const float* x, const float* w, int64_t rows, int n, float eps) {
    __shared__ float red[4];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + r * n;
        float* orow = out + r * n;
        float ss = 0.0f;
        for (int i = threadIdx.x; i < n; i += 256) ss += xr[i] * xr[i];
        const float tot = block_reduce<4>(ss, OpAdd(), red);
        const float rs = rsqrtf(tot / static_cast<float>(n) + eps);
        for (int i = threadIdx.x; i < n; i += 256) orow[i] = (w[i] * xr[i]) * rs;
        __syncthreads();
    }
}

}  // namespace

int rms_norm_rows_launch(float* out, const float* x, const float* w, int64_t rows, int n,
                         float eps, hipStream_t s) {
    if (!out || !x || !w || rows < 0 || n <= 0) return FENCE_ERROR_INVALID_VALUE;
    if (!aligned(out, 4) || !aligned(x, 4) || !aligned(w, 4)) return FENCE_ERROR_INVALID_VALUE;
    if (rows == 0) return FENCE_SUCCESS;
    const unsigned grid = grid_1d(rows, 1, 1 << 20);
    const bool vec = (n % 4 == 0) && aligned(out, 16) && aligned(x, 16) && aligned(w, 16);
    unsigned threads = 0;
    int vpt = 0;
    if (vec && plan_row(rows, n / 4, FENCE_RMS_VPT, 8, &threads, &vpt)) {
        if (vpt <= 2)
            return launch(rms_rows_vec_kernel<2>, dim3(grid), dim3(threads), 0, s, out, x, w, rows,
                          n, vpt, eps);
        return launch(rms_rows_vec_kernel<8>, dim3(grid), dim3(threads), 0, s, out, x, w, rows, n,
                      vpt, eps);
    }
    return launch(rms_rows_scalar_kernel, dim3(grid), dim3(256), 0, s, out, x, w, rows, n, eps);
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
