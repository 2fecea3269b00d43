// softmax.hip -- row softmax and causal softmax on gfx950.
//
// Follows softmax, src/kernels/ops.cuh:207-246, and the decode-attention
// softmax of gqa_attention_kernel, ops.cuh:357-391:
//   m = max(-1e30f, x_i);  e_i = expf(x_i - m);  x_i = e_i * (1.0f / sum e).
// The reference makes five global passes over the row (read for max,
// read+write exp, read+write scale).  Here a row is read once into VGPRs
// with 128-bit non-temporal loads, max and sum are DPP/readlane reductions
// (plus one LDS exchange when a row spans several waves), and the row is
// written once.  A row gets TPR lanes holding ~2 float4 each (generic) or ~4
// (causal, whose rows are short on average); rows of up to 256 lanes are
// packed several to a 256-thread workgroup.  All loads of a lane are issued
// before any of them is consumed.  e^x comes from exp_hw (common.hpp): the
// hardware base-2 exponential, within ~1e-6 relative of expf for the scores'
// range (x - m <= 0; masked -inf keys give exactly 0).
// Causal form: query i of sq sees keys 0 .. i + (sk - sq).  Keys past that
// bound are not read and are written as exactly 0.
#include "common.hpp"

#include <cmath>

#ifndef FENCE_SOFTMAX_VPT
#define FENCE_SOFTMAX_VPT 2
#endif
#ifndef FENCE_SOFTMAX_CAUSAL_VPT
#define FENCE_SOFTMAX_CAUSAL_VPT 4
#endif

namespace fence {
namespace {

constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ float max4(f4 v) { return fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)); }

__device__ __forceinline__ int row_valid(int64_t r, int n, int causal, int sq, int shift) {
    if (!causal) return n;
    int v = static_cast<int>(r % sq) + 1 + shift;
    return v < 0 ? 0 : (v > n ? n : v);
}

// TPR lanes per row (64, 128 or 256: 256/TPR rows per workgroup; 0: one row
// per workgroup of blockDim lanes, up to 1024).  MAXV float4 registers per
// lane, `vpt` of them used.
template <int MAXV, int TPR>
__global__ __launch_bounds__(TPR == 0 ? 1024 : 256) void softmax_vec_kernel(
    float* x, int64_t rows, int n, int64_t ld, int causal, int sq, int shift, int vpt) {
    constexpr int BLOCK = TPR == 0 ? 0 : 256;
    constexpr int RPB = TPR == 0 ? 1 : BLOCK / TPR;
    constexpr int WPR = TPR == 0 ? 0 : TPR / kWave;
    __shared__ float red_max[16];
    __shared__ float red_sum[16];
    const int tpr = TPR == 0 ? static_cast<int>(blockDim.x) : TPR;
    const int lt = threadIdx.x % tpr;
    const int sub = threadIdx.x / tpr;

    for (int64_t r0 = static_cast<int64_t>(blockIdx.x) * RPB; r0 < rows;
         r0 += static_cast<int64_t>(gridDim.x) * RPB) {
        const int64_t r = r0 + sub;
        const bool live = r < rows;  // uniform per row group
        float* row = x + (live ? r : 0) * ld;
        const int valid = live ? row_valid(r, n, causal, sq, shift) : 0;

        f4 v[MAXV];
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            const int e0 = 4 * (lt + j * tpr);
            v[j] = f4(kNegInf);
            if (j < vpt && e0 < valid) {
                if (e0 + 4 <= valid) {
                    v[j] = ld4<true>(row + e0);
                } else {
                    v[j].x = row[e0];
                    if (e0 + 1 < valid) v[j].y = row[e0 + 1];
                    if (e0 + 2 < valid) v[j].z = row[e0 + 2];
                }
            }
        }
        float m = -1e30f;
#pragma unroll
        for (int j = 0; j < MAXV; ++j) m = fmaxf(m, max4(v[j]));  // unloaded slots hold -inf
        if constexpr (TPR == 0) m = block_reduce_dyn(m, OpMax(), red_max);
        else m = row_reduce<WPR>(m, OpMax(), red_max);

        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < MAXV; ++j) {
            // whole chunk j of this row beyond the causal bound: nothing to do
            if (j < vpt && 4 * j * tpr < valid) {
                v[j].x = exp_hw(v[j].x - m);
                v[j].y = exp_hw(v[j].y - m);
                v[j].z = exp_hw(v[j].z - m);
                v[j].w = exp_hw(v[j].w - m);
                s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
            }
        }
        if constexpr (TPR == 0) s = block_reduce_dyn(s, OpAdd(), red_sum);
        else s = row_reduce<WPR>(s, OpAdd(), red_sum);
        const float inv = 1.0f / s;

        if (live) {
#pragma unroll
            for (int j = 0; j < MAXV; ++j) {
                const int e0 = 4 * (lt + j * tpr);
                if (j < vpt && e0 < n) {
                    f4 o;
                    o.x = (e0 + 0 < valid) ? v[j].x * inv : 0.0f;
                    o.y = (e0 + 1 < valid) ? v[j].y * inv : 0.0f;
                    o.z = (e0 + 2 < valid) ? v[j].z * inv : 0.0f;
                    o.w = (e0 + 3 < valid) ? v[j].w * inv : 0.0f;
                    if (e0 + 4 <= n) {
                        st4<true>(row + e0, o);
                    } else {
                        row[e0] = o.x;
                        if (e0 + 1 < n) row[e0 + 1] = o.y;
                        if (e0 + 2 < n) row[e0 + 2] = o.z;
                    }
                }
            }
        }
        if (TPR == 0 || WPR > 1) __syncthreads();  // red_max / red_sum are rewritten next row
    }
}

// Any n and alignment: one workgroup per row, three reads and one write.
__global__ __launch_bounds__(256) void softmax_scalar_kernel(float* x, int64_t rows, int n,
                                                             int64_t ld, int causal, int sq,
                                                             int shift) {
    __shared__ float red[4];
    for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
        float* row = x + r * ld;
        const int valid = row_valid(r, n, causal, sq, shift);
        float m = -1e30f;
        for (int i = threadIdx.x; i < valid; i += 256) m = fmaxf(m, row[i]);
        m = block_reduce<4>(m, OpMax(), red);
        __syncthreads();
        float s = 0.0f;
        for (int i = threadIdx.x; i < valid; i += 256) s += exp_hw(row[i] - m);
        s = block_reduce<4>(s, OpAdd(), red);
        const float inv = 1.0f / s;
        for (int i = threadIdx.x; i < n; i += 256) row[i] = (i < valid) ? exp_hw(row[i] - m) * inv : 0.0f;
        __syncthreads();
    }
}

template <int MAXV>
int launch_tpr(unsigned tpr, float* x, int64_t rows, int n, int64_t ld, int causal, int sq,
               int shift, int vpt, hipStream_t s) {
    switch (tpr) {
        case 64:
            return launch(softmax_vec_kernel<MAXV, 64>, dim3(grid_1d(rows, 4, 1 << 20)), dim3(256), 0,
                          s, x, rows, n, ld, causal, sq, shift, vpt);
        case 128:
            return launch(softmax_vec_kernel<MAXV, 128>, dim3(grid_1d(rows, 2, 1 << 20)), dim3(256), 0,
                          s, x, rows, n, ld, causal, sq, shift, vpt);
        case 256:
            return launch(softmax_vec_kernel<MAXV, 256>, dim3(grid_1d(rows, 1, 1 << 20)), dim3(256), 0,
                          s, x, rows, n, ld, causal, sq, shift, vpt);
        default:
            return launch(softmax_vec_kernel<MAXV, 0>, dim3(grid_1d(rows, 1, 1 << 20)), dim3(tpr), 0,
                          s, x, rows, n, ld, causal, sq, shift, vpt);
    }
}

int softmax_launch(float* x, int64_t rows, int n, int64_t ld, int causal, int sq, int shift,
                   hipStream_t s) {
    const bool vec = aligned(x, 16) && (ld % 4 == 0);
    unsigned tpr = 0;
    int vpt = 0;
    const int target = causal ? FENCE_SOFTMAX_CAUSAL_VPT : FENCE_SOFTMAX_VPT;
    if (vec && plan_row(rows, (n + 3) / 4, target, 16, &tpr, &vpt)) {
        if (tpr > 64 && tpr < 128) tpr = 128;  // rows sharing a workgroup take 64/128/256 lanes
        else if (tpr > 128 && tpr < 256) tpr = 256;
        vpt = static_cast<int>(((n + 3) / 4 + tpr - 1) / tpr);
        if (vpt <= 2) return launch_tpr<2>(tpr, x, rows, n, ld, causal, sq, shift, vpt, s);
        if (vpt <= 4) return launch_tpr<4>(tpr, x, rows, n, ld, causal, sq, shift, vpt, s);
        if (vpt <= 8) return launch_tpr<8>(tpr, x, rows, n, ld, causal, sq, shift, vpt, s);
        return launch_tpr<16>(tpr, x, rows, n, ld, causal, sq, shift, vpt, s);
    }
    return launch(softmax_scalar_kernel, dim3(grid_1d(rows, 1, 1 << 20)), dim3(256), 0, s, x, rows,
                  n, ld, causal, sq, shift);
}

}  // namespace
}  // namespace fence

extern "C" int fence_softmax(float* x, int n, hipStream_t stream) {
    if (!x || n <= 0 || !fence::aligned(x, 4)) return FENCE_ERROR_INVALID_VALUE;
    return fence::softmax_launch(x, 1, n, n, 0, 1, 0, stream);
}

extern "C" int fence_softmax_rows(float* x, int64_t rows, int n, int64_t ld, hipStream_t stream) {
    if (!x || rows < 0 || n <= 0 || ld < n || !fence::aligned(x, 4)) return FENCE_ERROR_INVALID_VALUE;
    if (rows == 0) return FENCE_SUCCESS;
    return fence::softmax_launch(x, rows, n, ld, 0, 1, 0, stream);
}

extern "C" int fence_softmax_causal(float* x, int64_t heads, int sq, int sk, hipStream_t stream) {
    if (!x || heads < 0 || sq <= 0 || sk <= 0 || !fence::aligned(x, 4)) return FENCE_ERROR_INVALID_VALUE;
    if (heads == 0) return FENCE_SUCCESS;
    return fence::softmax_launch(x, heads * sq, sk, sk, 1, sq, sk - sq, stream);
}
