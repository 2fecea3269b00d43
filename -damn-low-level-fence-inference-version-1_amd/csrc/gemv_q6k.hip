// gemv_q6k.hip -- Q6_K matrix-vector product y = W x (+ bias) on gfx950: the
// projections of a decode step (attention q/k/v/o, FFN gate/up/down).
//
// Follows gemv_q6k / gemv_q6k_bias, src/kernels/gemv_q6k.cuh:44-151, on the
// block layout of src/kernels/q6k_types.h:24-35 (ql[128], qh[64], int8
// scales[16], fp16 d; 210 bytes per 256 weights) with x in binary16:
//   y[r] = sum_b d_b * sum_i scales_b[i/16] * (q6_b[i] - 32) * x[256b + i]
// where element i = 128h + 32c + l of a block has its low nibble in
// ql[64h + l + 32(c&1)] (high nibble for c >= 2) and its top two bits at bit
// 2c of qh[32h + l] (src/kernels/q6k_dot.cuh:35-64).
//
// Work split.  Sixteen lanes share a block: lane (h, j) of a block owns
// l = 4j..4j+3 of half h in all four columns c -- 16 weights that come from
// one ql dword at 64h + 4j, one at 64h + 32 + 4j and one qh dword at
// 128 + 32h + 4j, with one scale per column, scales[8h + 2c + j/4].  A wave
// covers four blocks per pass.  Each lane rebuilds a column's four quants with
// byte-parallel bit operations, turns each pair into binary16 values
// 1024 + q with one v_perm_b32 (0x64 above each quant byte), and multiplies
// them with x's binary16 pairs in v_dot2c_f32_f16, starting each column's sum
// at -1056 * (sum of its four x) -- precomputed once per wave, since a lane's
// x never changes -- which leaves sum (q - 32) * x.  That is about two VALU
// operations per weight instead of four.
//
// Memory.  Blocks are only 2-byte aligned (210 = 2 * 105).  One wave stages
// its segment of a row (up to 16 blocks) into its own LDS buffer with
// aligned 128-bit non-temporal loads over the 16-byte chunks that cover it,
// then reads each lane's dwords back from LDS realigned with v_alignbyte.
// Staging needs W 16-byte aligned and M * K/256 a multiple of 8 (so the whole
// matrix is a whole number of chunks and no chunk extends past it); otherwise
// a direct kernel reads the same dwords from global memory.  Rows of more than
// 16 blocks are split over 2 or 4 waves of the workgroup, whose partial sums
// meet in LDS.  The lane's x values (16 per pass) stay in VGPRs for all rows.
#include <atomic>

#include "common.hpp"

// 1: a wave issues the next row segment's loads before computing the current one.
#ifndef FENCE_GEMV_Q6K_PREFETCH
#define FENCE_GEMV_Q6K_PREFETCH 0
#endif

namespace fence {
namespace {

constexpr int kThreads = 256;
constexpr int kBlockBytes = 210;
constexpr int kMaxSegBlocks = 16;  // blocks of one row staged by one wave

// The 16 quants (0..63) of one lane of one block, one byte each: w[c] holds
// column c's four (l = 4j .. 4j+3).
struct Q6Lane {
    uint32_t w[4];
};

__device__ __forceinline__ Q6Lane q6_unpack(uint32_t a, uint32_t b, uint32_t c) {
    constexpr uint32_t kNib = 0x0F0F0F0Fu;    // low nibble of every byte
    constexpr uint32_t kCrumb = 0x30303030u;  // bits 4..5: the high two bits
    Q6Lane r;
    r.w[0] = (a & kNib) | ((c << 4) & kCrumb);
    r.w[1] = (b & kNib) | ((c << 2) & kCrumb);
    r.w[2] = ((a >> 4) & kNib) | (c & kCrumb);
    r.w[3] = ((b >> 4) & kNib) | ((c >> 2) & kCrumb);
    return r;
}

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Two quants as binary16 pairs 1024 + q (exact: 0x64 above each quant byte).
__device__ __forceinline__ h2 q6_pair(uint32_t w, uint32_t sel) {
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(w, 0x64646464u, sel));
}

// Per column of a lane: the bias -1056 * (x0 + x1 + x2 + x3).  A column's
// sum over (1024 + q) * x then starts from it, which leaves
// sum (q - 32) * x: the -32 of the format and the 1024 of the binary16
// encoding cancel exactly when x is a unit vector, and otherwise to within
// fp32 rounding of terms of size 1056 |x|.
__device__ __forceinline__ float q6_col_bias(uint32_t x01, uint32_t x23) {
    const h2 a = __builtin_bit_cast(h2, x01), b = __builtin_bit_cast(h2, x23);
    return -1056.0f * ((static_cast<float>(a.x) + static_cast<float>(a.y)) +
                       (static_cast<float>(b.x) + static_cast<float>(b.y)));
}

// d * sum_c sc_c * sum_k (q - 32) * x over the lane's 16 weights of one block,
// each pair of weights one v_dot2c_f32_f16.
__device__ __forceinline__ float q6_lane_dot(const Q6Lane& q, const uint32_t* xh, const float* kb, const int* sc,
                                             float d) {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        float p = __builtin_amdgcn_fdot2(q6_pair(q.w[c], 0x00050004u), __builtin_bit_cast(h2, xh[2 * c]), kb[c],
                                         false);
        p = __builtin_amdgcn_fdot2(q6_pair(q.w[c], 0x00070006u), __builtin_bit_cast(h2, xh[2 * c + 1]), p, false);
        acc = __builtin_fmaf(static_cast<float>(sc[c]), p, acc);
    }
    return d * acc;
}

__device__ __forceinline__ float wave_sum(float v) { return wave_reduce(v, OpAdd{}); }

// The segment [b0, b1) of the row's blocks a wave handles when WPR waves
// share a row: an even split.
__device__ __forceinline__ void segment(int nb, int seg, int wpr, int* b0, int* b1) {
    *b0 = (nb * seg) / wpr;
    *b1 = (nb * (seg + 1)) / wpr;
}

template <int PASSES>
__device__ __forceinline__ void load_x(uint32_t (&xh)[PASSES][8], float (&kb)[PASSES][4], const uint16_t* x16,
                                       int b0, int b1, int bslot, int h, int j) {
    const bool vec = (reinterpret_cast<uintptr_t>(x16) & 7) == 0;
#pragma unroll
    for (int p = 0; p < PASSES; ++p) {
        const int b = b0 + 4 * p + bslot;
        const bool on = b < b1;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int e = 256 * (on ? b : b0) + 128 * h + 32 * c + 4 * j;  // inside x either way
            uint32_t lo, hi;
            if (vec) {
                const uint2 v = *reinterpret_cast<const uint2*>(x16 + e);
                lo = v.x;
                hi = v.y;
            } else {
                lo = x16[e] | (static_cast<uint32_t>(x16[e + 1]) << 16);
                hi = x16[e + 2] | (static_cast<uint32_t>(x16[e + 3]) << 16);
            }
            xh[p][2 * c] = on ? lo : 0u;  // binary16 zeros: a masked block adds 0
            xh[p][2 * c + 1] = on ? hi : 0u;
            kb[p][c] = q6_col_bias(xh[p][2 * c], xh[p][2 * c + 1]);
        }
    }
}

// Staged kernel.  WPR waves per row (1, 2 or 4), each over at most 4 * PASSES
// <= 16 blocks.  LDS: 4 wave buffers of kSegBytes + red[4].
template <int PASSES, int WPR, bool PF>
__global__ __launch_bounds__(kThreads) void gemv_q6k_staged_kernel(float* __restrict__ y,
                                                                   const uint8_t* __restrict__ W,
                                                                   const uint16_t* __restrict__ x16,
                                                                   const float* __restrict__ bias, int M,
                                                                   int nb) {
    constexpr int kSegBytes = 4 * PASSES * kBlockBytes + 32;  // + alignment slack
    constexpr int kBufBytes = (kSegBytes + 15) / 16 * 16;
    constexpr int kChunkSlots = (kSegBytes / 16 + kWave - 1) / kWave;
    constexpr int kRowsPerGroup = 4 / WPR;
    constexpr uint32_t kPassBytes = 4 * kBlockBytes;  // 840: a multiple of 4
    __shared__ __align__(16) uint8_t lds[4 * kBufBytes];
    __shared__ float red[4];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));  // wave-uniform
    const int seg = wid % WPR;
    const int rslot = wid / WPR;
    uint8_t* buf = lds + wid * kBufBytes;
    const int bslot = lane >> 4, h = (lane >> 3) & 1, j = lane & 7;
    int b0, b1;
    segment(nb, seg, WPR, &b0, &b1);
    const int64_t row_bytes = static_cast<int64_t>(nb) * kBlockBytes;

    uint32_t xh[PASSES][8];
    float kb[PASSES][4];
    load_x<PASSES>(xh, kb, x16, b0, b1, bslot, h, j);
    bool on[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) on[p] = b0 + 4 * p + bslot < b1;
    const uint32_t lane_ql = 64 * h + 4 * j;         // ql dword of the lane in its block
    const uint32_t lane_qh = 128 + 32 * h + 4 * j;   // qh dword
    const uint32_t lane_sc = 192 + 8 * h + (j >> 2);  // column 0's scale byte
    const uint32_t blk_off = static_cast<uint32_t>(bslot) * kBlockBytes;

    // The 16-byte chunks covering group g's segment: [a0, a0 + 16 * nch).
    auto seg_of = [&](int64_t g, int64_t* a0, int* nch, uint32_t* delta) {
        const int64_t r = g * kRowsPerGroup + rslot;
        const int64_t rr = r < M ? r : M - 1;  // clamped: a prefetch past the last row stays inside W
        const int64_t start = rr * row_bytes + static_cast<int64_t>(b0) * kBlockBytes;
        const int64_t end = rr * row_bytes + static_cast<int64_t>(b1) * kBlockBytes;
        *a0 = start & ~int64_t(15);
        *nch = static_cast<int>((end - *a0 + 15) >> 4);
        *delta = static_cast<uint32_t>(start - *a0);
    };
    // Loads of one segment's chunks: clamped and opaque offsets, so every
    // load is issued unconditionally in scalar-base + VGPR-offset form.
    auto load_seg = [&](int64_t a0, int nch, u4* ch) {
        const uint8_t* src = W + a0;
#pragma unroll
        for (int k = 0; k < kChunkSlots; ++k) {
            const int cc = lane + kWave * k;
            uint32_t off = 16u * static_cast<uint32_t>(cc < nch ? cc : 0);
            asm volatile("" : "+v"(off));
            ch[k] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(src + off));
        }
    };
    u4 ch[kChunkSlots];
    int64_t a0n;
    int nchn;
    uint32_t deltan;
    if constexpr (PF) {
        seg_of(blockIdx.x, &a0n, &nchn, &deltan);
        load_seg(a0n, nchn, ch);
    }
    for (int64_t g = blockIdx.x; g * kRowsPerGroup < M; g += gridDim.x) {
        const int64_t r = g * kRowsPerGroup + rslot;  // wave-uniform
        float part = 0.0f;
        int64_t a0;
        int nch;
        uint32_t delta;
        if constexpr (PF) {
            a0 = a0n, nch = nchn, delta = deltan;
        } else {
            seg_of(g, &a0, &nch, &delta);
            load_seg(a0, nch, ch);
        }
        if (r < M) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < kChunkSlots; ++k) {
                const int cc = lane + kWave * k;
                // a lane past the segment's last chunk stores into the slack
                // at the buffer's end, which holds no block data
                const uint32_t dst = cc < nch ? 16u * cc : static_cast<uint32_t>(kBufBytes - 16);
                *reinterpret_cast<u4*>(buf + dst) = ch[k];
            }
        }
        if constexpr (PF) {
            // the next group's loads fly while this one is computed from LDS
            seg_of(g + gridDim.x, &a0n, &nchn, &deltan);
            load_seg(a0n, nchn, ch);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (r < M) {
            // The lane's block starts at `base` in the buffer for pass 0 and
            // 840 bytes later per pass; every dword it reads has the same
            // offset mod 4, so one aligned base and one shift serve them all.
            const uint32_t base = delta + blk_off;
            const uint32_t sh = base & 3u;
            const uint8_t* ab = buf + (base & ~3u);
            const uint8_t* bb = buf + base;
#pragma unroll
            for (int p = 0; p < PASSES; ++p) {
                // masked passes read a staged block too (inside the buffer) and are dropped
                const uint32_t* wa = reinterpret_cast<const uint32_t*>(ab + p * kPassBytes + lane_ql);
                const uint32_t* wb = reinterpret_cast<const uint32_t*>(ab + p * kPassBytes + lane_ql + 32);
                const uint32_t* wc = reinterpret_cast<const uint32_t*>(ab + p * kPassBytes + lane_qh);
                const uint32_t a = __builtin_amdgcn_alignbyte(wa[1], wa[0], sh);
                const uint32_t bq = __builtin_amdgcn_alignbyte(wb[1], wb[0], sh);
                const uint32_t c = __builtin_amdgcn_alignbyte(wc[1], wc[0], sh);
                const int8_t* scb = reinterpret_cast<const int8_t*>(bb + p * kPassBytes + lane_sc);
                int sc[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) sc[q] = scb[2 * q];
                const uint16_t dbits = *reinterpret_cast<const uint16_t*>(bb + p * kPassBytes + 208);
                const float d = static_cast<float>(__builtin_bit_cast(_Float16, dbits));
                const float v = q6_lane_dot(q6_unpack(a, bq, c), xh[p], kb[p], sc, d);
                part += on[p] ? v : 0.0f;
            }
            part = wave_sum(part);
        }
        if constexpr (WPR == 1) {
            if (r < M && lane == 0) y[r] = bias ? part + bias[r] : part;
        } else {
            if (lane == 0) red[wid] = part;
            __syncthreads();
            if (seg == 0 && lane == 0 && r < M) {
                float t = red[wid];
#pragma unroll
                for (int s = 1; s < WPR; ++s) t += red[wid + s];
                y[r] = bias ? t + bias[r] : t;
            }
            __syncthreads();  // red[] is rewritten by the next group
        }
    }
}

// Direct kernel for any alignment and any K: the same lanes, the dwords read
// straight from global memory (two aligned dwords each, realigned).
__global__ __launch_bounds__(kThreads) void gemv_q6k_direct_kernel(float* __restrict__ y,
                                                                   const uint8_t* __restrict__ W,
                                                                   const uint16_t* __restrict__ x16,
                                                                   const float* __restrict__ bias, int M,
                                                                   int nb) {
    const int lane = threadIdx.x & (kWave - 1);
    const int bslot = lane >> 4, h = (lane >> 3) & 1, j = lane & 7;
    const int64_t row_bytes = static_cast<int64_t>(nb) * kBlockBytes;
    const int64_t wave = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) / kWave;
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * (kThreads / kWave);
    for (int64_t r = wave; r < M; r += nwaves) {
        float part = 0.0f;
        for (int b0 = 0; b0 < nb; b0 += 4) {
            const int b = b0 + bslot;
            if (b < nb) {
                const uint8_t* blk = W + r * row_bytes + static_cast<int64_t>(b) * kBlockBytes;
                auto rd = [&](int off) {
                    const uint8_t* p = blk + off;
                    const uint32_t* w = reinterpret_cast<const uint32_t*>(reinterpret_cast<uintptr_t>(p) & ~uintptr_t(3));
                    const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 3);
                    // both dwords lie inside the 210-byte block for every offset used
                    return sh ? __builtin_amdgcn_alignbyte(w[1], w[0], sh) : w[0];
                };
                const uint32_t a = rd(64 * h + 4 * j), bq = rd(64 * h + 32 + 4 * j), c = rd(128 + 32 * h + 4 * j);
                int sc[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) sc[q] = static_cast<int8_t>(blk[192 + 8 * h + (j >> 2) + 2 * q]);
                const uint16_t dbits = static_cast<uint16_t>(blk[208] | (blk[209] << 8));
                uint32_t xh[8];
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) {
                    const int e = 256 * b + 128 * h + 32 * cc + 4 * j;
                    xh[2 * cc] = x16[e] | (static_cast<uint32_t>(x16[e + 1]) << 16);
                    xh[2 * cc + 1] = x16[e + 2] | (static_cast<uint32_t>(x16[e + 3]) << 16);
                }
                float kbc[4];
#pragma unroll
                for (int cc = 0; cc < 4; ++cc) kbc[cc] = q6_col_bias(xh[2 * cc], xh[2 * cc + 1]);
                const float d = static_cast<float>(__builtin_bit_cast(_Float16, dbits));
                part += q6_lane_dot(q6_unpack(a, bq, c), xh, kbc, sc, d);
            }
        }
        part = wave_sum(part);
        if (lane == 0) y[r] = bias ? part + bias[r] : part;
    }
}

template <class Kernel>
int launch_grid(Kernel kernel, int64_t groups, float* y, const uint8_t* W, const uint16_t* x, const float* bias,
                int M, int nb, hipStream_t s) {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_status(e);
    if (dev < 0 || dev >= 64) return FENCE_ERROR_INVALID_VALUE;
    int g = cache[dev].load(std::memory_order_relaxed);
    if (g == 0) {
        int cus = 0, per_cu = 0;
        if (hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev); e != hipSuccess)
            return hip_status(e);
        if (hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, 0);
            e != hipSuccess)
            return hip_status(e);
        g = cus * (per_cu > 0 ? per_cu : 1);
        cache[dev].store(g, std::memory_order_relaxed);
    }
    const unsigned grid = static_cast<unsigned>(groups < g ? groups : g);
    return launch(kernel, dim3(grid), dim3(kThreads), 0, s, y, W, x, bias, M, nb);
}

template <int PASSES, int WPR>
int launch_staged(float* y, const uint8_t* W, const uint16_t* x, const float* bias, int M, int nb, hipStream_t s) {
    constexpr int rows_per_group = 4 / WPR;
    return launch_grid(gemv_q6k_staged_kernel<PASSES, WPR, FENCE_GEMV_Q6K_PREFETCH != 0>,
                       (M + rows_per_group - 1) / rows_per_group, y, W, x, bias, M, nb, s);
}

int gemv_q6k_launch(float* y, const void* Wv, const void* xv, const float* bias, int M, int K, hipStream_t s) {
    if (M < 0 || K < 0 || (K % 256) != 0) return FENCE_ERROR_INVALID_VALUE;
    if (M == 0) return FENCE_SUCCESS;
    if (K == 0 || !y || !Wv || !xv) return FENCE_ERROR_INVALID_VALUE;
    const uint8_t* W = static_cast<const uint8_t*>(Wv);
    const uint16_t* x = static_cast<const uint16_t*>(xv);
    if (!aligned(W, 2) || !aligned(x, 2) || !aligned(y, 4) || (bias && !aligned(bias, 4)))
        return FENCE_ERROR_INVALID_VALUE;
    const int nb = K / 256;
    const bool staged = aligned(W, 16) && (static_cast<int64_t>(M) * nb) % 8 == 0 && nb <= 4 * kMaxSegBlocks;
    if (staged) {
        if (nb <= 4) return launch_staged<1, 1>(y, W, x, bias, M, nb, s);
        if (nb <= 8) return launch_staged<2, 1>(y, W, x, bias, M, nb, s);
        if (nb <= 12) return launch_staged<3, 1>(y, W, x, bias, M, nb, s);
        if (nb <= 16) return launch_staged<4, 1>(y, W, x, bias, M, nb, s);
        if (nb <= 24) return launch_staged<3, 2>(y, W, x, bias, M, nb, s);
        if (nb <= 32) return launch_staged<4, 2>(y, W, x, bias, M, nb, s);
        if (nb <= 48) return launch_staged<3, 4>(y, W, x, bias, M, nb, s);
        return launch_staged<4, 4>(y, W, x, bias, M, nb, s);
    }
    return launch_grid(gemv_q6k_direct_kernel, (static_cast<int64_t>(M) + 3) / 4, y, W, x, bias, M, nb, s);
}

}  // namespace
}  // namespace fence

extern "C" int fence_gemv_q6k(const void* W, const void* x, float* y, int M, int K, hipStream_t stream) {
    return fence::gemv_q6k_launch(y, W, x, nullptr, M, K, stream);
}

extern "C" int fence_gemv_q6k_bias(const void* W, const void* x, const float* bias, float* y, int M, int K,
                                   hipStream_t stream) {
    if (!bias) return FENCE_ERROR_INVALID_VALUE;
    return fence::gemv_q6k_launch(y, W, x, bias, M, K, stream);
}
