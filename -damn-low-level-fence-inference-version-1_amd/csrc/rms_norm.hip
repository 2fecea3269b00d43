// rms_norm.hip -- row RMSNorm on gfx950.
//
// Follows rms_norm, src/kernels/ops.cuh:17-51:
//   r = rsqrt(sum(x^2) / n + eps);  out[i] = (w[i] * x[i]) * r.
// The reference runs one 1024-thread block and reads x twice.  Here one
// workgroup owns one row, the row is read once with 128-bit loads and kept
// in VGPRs, the sum of squares is reduced with DPP inside each wave and one
// LDS exchange across waves, and the normalised row is written from the
// registers.  out may equal x: every element is read before the barrier in
// the reduction and written after it.
#include "common.hpp"

namespace fence {
namespace {

template <int NWAVES, int MAXV>
__global__ __launch_bounds__(NWAVES * kWave) void rms_rows_vec_kernel(
    float* out, const float* x, const float* w, int64_t rows, int n, int vpt, float eps) {
    constexpr int T = NWAVES * kWave;
    __shared__ float red[NWAVES];
    const int n4 = n >> 2;
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        const float* xr = x + r * n;
        float* orow = out + r * n;
        f4 v[MAXV];
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int f = threadIdx.x + j * T;
            if (j < vpt && f < n4) {
                v[j] = ld4<false>(xr + 4 * f);
                ss += dot4(v[j]);
            }
        }
        const float tot = block_reduce<NWAVES>(ss, OpAdd(), red);
        const float rs = rsqrtf(tot / static_cast<float>(n) + eps);
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int f = threadIdx.x + j * T;
            if (j < vpt && f < n4) {
                const f4 wv = ld4<false>(w + 4 * f);
                st4<false>(orow + 4 * f, (wv * v[j]) * rs);
            }
        }
        if constexpr (NWAVES > 1) __syncthreads();  // red[] is rewritten by the next row
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

template <int NWAVES, int MAXV>
int rows_vec(float* out, const float* x, const float* w, int64_t rows, int n, int vpt, float eps,
             hipStream_t s) {
    const unsigned grid = grid_1d(rows, 1, 1 << 20);
    return launch(rms_rows_vec_kernel<NWAVES, MAXV>, dim3(grid), dim3(NWAVES * kWave), 0, s, out, x,
                  w, rows, n, vpt, eps);
}

}  // namespace

int rms_norm_rows_launch(float* out, const float* x, const float* w, int64_t rows, int n,
                         float eps, hipStream_t s) {
    if (!out || !x || !w || rows < 0 || n <= 0) return FENCE_ERROR_INVALID_VALUE;
    if (!aligned(out, 4) || !aligned(x, 4) || !aligned(w, 4)) return FENCE_ERROR_INVALID_VALUE;
    if (rows == 0) return FENCE_SUCCESS;
    const bool vec = (n % 4 == 0) && aligned(out, 16) && aligned(x, 16) && aligned(w, 16);
    const int n4 = n / 4;
    if (vec) {
        if (n4 <= kWave * 4) return rows_vec<1, 4>(out, x, w, rows, n, (n4 + 63) / 64, eps, s);
        const int v256 = (n4 + 255) / 256;
        if (v256 <= 4) return rows_vec<4, 4>(out, x, w, rows, n, v256, eps, s);
        if (v256 <= 8) return rows_vec<4, 8>(out, x, w, rows, n, v256, eps, s);
        if (v256 <= 16) return rows_vec<4, 16>(out, x, w, rows, n, v256, eps, s);
        const int v1024 = (n4 + 1023) / 1024;
        if (v1024 <= 16) return rows_vec<16, 16>(out, x, w, rows, n, v1024, eps, s);
    }
    const unsigned grid = grid_1d(rows, 1, 1 << 20);
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
