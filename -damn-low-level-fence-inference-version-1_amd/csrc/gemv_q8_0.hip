// gemv_q8_0.hip -- Q8_0 matrix-vector product y = W x on gfx950 (the tied
// LM head of a decode step).
//
// Follows gemv_q8_0, src/kernels/gemv_q8_0.cuh:38-104: W holds M rows of K/32
// Q8_0 blocks (fp16 scale d, then 32 int8 qs; 34 bytes, src/kernels/
// q8_0_types.h:8-17), x and y are fp32, and
//   y[r] = sum_b d_b * sum_i qs_b[i] * x[32b + i].
//
// The op reads every byte of W once per call and does two VALU operations per
// byte (int8 -> fp32 convert, fma), so it is HBM-bound.  One wave computes a
// whole row: lane l owns the 8-weight quarters q = l, l+64, l+128, ... of
// every row (a quarter of block b = q/4 sits at byte 34b + 2 + 8(q%4)), so the
// 8 x values a quarter multiplies stay in that lane's VGPRs for all the rows
// the wave visits, and x is read from memory once per wave.  Per row a lane
// issues all its 8-byte quarter loads and 2-byte scale loads before consuming
// any (the quarters of one wave cover 16 consecutive blocks, 544 contiguous
// bytes, so each load instruction coalesces into a few cache lines; the four
// lanes of a block read the same scale from the same line), forms
// each block's 32-product sum across its quad of lanes (two DPP adds), adds
// d * block_sum on the quad's first lane, and the row sum is one wave
// reduction.
// Waves stride over rows, so concurrently running waves stream neighbouring
// rows.  W is read with non-temporal loads: it is larger than the L2 and the
// MALL and is not re-read within a call.
#include <atomic>

#include "common.hpp"

// Rows whose loads one wave issues together, and the most workgroups (of 4
// waves) per CU in the grid; the grid never exceeds what is resident at once.
// FENCE_GEMV_Q8_WG_PER_CU, when defined, sets the staged kernel's cap for
// every K (otherwise q8_staged_wg_per_cu below).
#ifndef FENCE_GEMV_Q8_ROWS
#define FENCE_GEMV_Q8_ROWS 1
#endif
#ifndef FENCE_GEMV_Q8_STAGED
#define FENCE_GEMV_Q8_STAGED 1
#endif
#ifndef FENCE_GEMV_Q8_PREFETCH
#define FENCE_GEMV_Q8_PREFETCH 1
#endif

namespace fence {
namespace {

constexpr int kGemvThreads = 256;  // 4 waves; up to 16 quarter slots (K <= 8192) keep x in VGPRs

typedef uint32_t u2a2 __attribute__((ext_vector_type(2), aligned(2)));

__device__ __forceinline__ float q8_quarter_dot(u2a2 q, const float* xs) {
    // 8 products accumulated with fused multiply-adds
    float p = static_cast<float>(static_cast<int8_t>(q.x & 0xFFu)) * xs[0];
    p = __builtin_fmaf(static_cast<float>(static_cast<int8_t>((q.x >> 8) & 0xFFu)), xs[1], p);
    p = __builtin_fmaf(static_cast<float>(static_cast<int8_t>((q.x >> 16) & 0xFFu)), xs[2], p);
    p = __builtin_fmaf(static_cast<float>(static_cast<int8_t>(q.x >> 24)), xs[3], p);
    p = __builtin_fmaf(static_cast<float>(static_cast<int8_t>(q.y & 0xFFu)), xs[4], p);
    p = __builtin_fmaf(static_cast<float>(static_cast<int8_t>((q.y >> 8) & 0xFFu)), xs[5], p);
    p = __builtin_fmaf(static_cast<float>(static_cast<int8_t>((q.y >> 16) & 0xFFu)), xs[6], p);
    return __builtin_fmaf(static_cast<float>(static_cast<int8_t>(q.y >> 24)), xs[7], p);
}

// The four lanes of an aligned quad hold the four quarters of one block:
// sum their partials so that, as in the reference, each block contributes
// d * (sum of its 32 products).  Non-finite scales then propagate exactly as
// the reference's d * block_sum does.
__device__ __forceinline__ float block_sum(float part) {
    part = part + dpp<kDppQuadXor1>(part);
    return part + dpp<kDppQuadXor2>(part);
}

__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Sum of one value per aligned quad over a wave, for values that are equal
// across each quad: the quad steps of the full reduction are skipped.
__device__ __forceinline__ float wave_sum_of_quads(float v) {
    v = v + dpp<kDppHalfMirror>(v);
    v = v + dpp<kDppMirror>(v);
    return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

// SLOTS quarters per lane with their x in VGPRs; ROWS rows' loads in flight
// per wave.  Slot s of lane l is quarter q = l + 64s: block (l >> 2) + 16s,
// quarter l & 3 of it, so its bytes lie exactly 544s after slot 0's.  FULL:
// K % 512 == 0, every slot is inside the row and needs no mask.  W must be
// 2-byte aligned.
template <int SLOTS, int ROWS, bool FULL>
__global__ __launch_bounds__(kGemvThreads) void gemv_q8_0_kernel(float* __restrict__ y,
                                                                 const uint8_t* __restrict__ W,
                                                                 const float* __restrict__ x,
                                                                 int M, int K) {
    const int lane = threadIdx.x & (kWave - 1);
    const int nq = K >> 3;
    const int64_t row_bytes = static_cast<int64_t>(K >> 5) * 34;
    constexpr uint32_t kSlotBytes = 16 * 34;
    const uint32_t d_off0 = 34 * static_cast<uint32_t>(lane >> 2);
    const uint32_t q_off0 = d_off0 + 2 + 8 * static_cast<uint32_t>(lane & 3);

    float xs[SLOTS][8];
    bool on[SLOTS];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int q = lane + kWave * s;
        on[s] = FULL || q < nq;
        const int qc = on[s] ? q : 0;  // a masked slot re-reads quarter 0: inside x
#pragma unroll
        for (int j = 0; j < 8; ++j) xs[s][j] = x[8 * qc + j];  // unconditional: no branch per load
        if constexpr (!FULL) {
#pragma unroll
            for (int j = 0; j < 8; ++j) xs[s][j] = on[s] ? xs[s][j] : 0.0f;
        }
    }

    // wave-uniform in an SGPR, so each row's base address is scalar and every
    // load is a 32-bit lane offset (plus an immediate) from it
    const int wave = __builtin_amdgcn_readfirstlane(
        static_cast<int>((blockIdx.x * static_cast<unsigned>(kGemvThreads) + threadIdx.x) / kWave));
    const int nwaves = static_cast<int>(gridDim.x * (kGemvThreads / kWave));
    for (int r0 = wave * ROWS; r0 < M; r0 += nwaves * ROWS) {
        // opaque each iteration, so the loads keep the scalar-base + VGPR-offset
        // form instead of 64-bit per-lane addresses hoisted out of the loop
        uint32_t qo = q_off0, dof = d_off0;
        asm volatile("" : "+v"(qo), "+v"(dof));
        u2a2 qv[ROWS][SLOTS];
        uint16_t dv[ROWS][SLOTS];
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            const int r = r0 + i < M ? r0 + i : M - 1;  // clamped: loads stay inside W
            const uint8_t* row = W + static_cast<int64_t>(r) * row_bytes;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                // a masked slot re-reads block 0 (quarter 0 and its scale), which
                // every row has; its product is discarded
                const uint32_t q_at = on[s] ? qo + kSlotBytes * s : 2u;
                const uint32_t d_at = on[s] ? dof + kSlotBytes * s : 0u;
                qv[i][s] = __builtin_nontemporal_load(reinterpret_cast<const u2a2*>(row + q_at));
                dv[i][s] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(row + d_at));
            }
        }
        // every load of the iteration is issued before the first is consumed
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            // Each lane of a quad holds the same d * block_sum, so the sum over
            // quads counts every block once.
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                const float bs = block_sum(q8_quarter_dot(qv[i][s], xs[s]));
                const float c = half_bits_to_float(dv[i][s]) * bs;
                if constexpr (FULL) acc += c;
                else acc += on[s] ? c : 0.0f;  // a masked slot adds exactly 0, even if d is inf/NaN
            }
            acc = wave_sum_of_quads(acc);
            if (lane == 0 && r0 + i < M) y[r0 + i] = acc;
        }
    }
}

// The same quarter computation, with each row staged through LDS: when a row
// is a whole number of 16-byte chunks (K % 256 == 0) and W is 16-byte
// aligned, the wave reads the row with aligned 128-bit loads (consecutive
// lanes, consecutive chunks: every load instruction covers 1 KiB of whole
// cache lines), writes it to its own LDS row buffer, and each lane then reads
// its 2-byte-aligned quarters from LDS as three dwords realigned with
// v_alignbyte.  One wave's LDS operations complete in order, so the next
// row's writes cannot overtake this row's reads.  LDS: 4 * row_bytes + 16
// bytes per workgroup; the 16 pad bytes take the unused third dword of the
// last quarter and the stores of lanes past the row's last chunk.  PF rows
// of loads are in flight while a row is computed (0: none; 2: two register
// buffers, refilled alternately).
template <int SLOTS, bool FULL, int PF>
__global__ __launch_bounds__(kGemvThreads) void gemv_q8_0_staged_kernel(float* __restrict__ y,
                                                                        const uint8_t* __restrict__ W,
                                                                        const float* __restrict__ x,
                                                                        int M, int K) {
    constexpr int kChunkSlots = (34 * SLOTS + kWave - 1) / kWave;  // 16-byte chunks per lane per row
    extern __shared__ __align__(16) uint8_t row_lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int nq = K >> 3;
    const int row_bytes = (K >> 5) * 34;
    const int nchunks = row_bytes >> 4;
    uint8_t* buf = row_lds + (threadIdx.x / kWave) * row_bytes;
    uint8_t* pad = row_lds + (kGemvThreads / kWave) * row_bytes;
    constexpr uint32_t kSlotBytes = 16 * 34;
    const uint32_t d_off0 = 34 * static_cast<uint32_t>(lane >> 2);
    const uint32_t q_off0 = d_off0 + 2 + 8 * static_cast<uint32_t>(lane & 3);
    const uint32_t q_base0 = q_off0 & ~3u;  // dword holding the quarter's first byte
    const uint32_t q_shift = q_off0 & 3u;   // 0 or 2: bytes to drop from it

    const int wave = __builtin_amdgcn_readfirstlane(
        static_cast<int>((blockIdx.x * static_cast<unsigned>(kGemvThreads) + threadIdx.x) / kWave));
    const int nwaves = static_cast<int>(gridDim.x * (kGemvThreads / kWave));
    // Loads of one row: clamped (inside the row) and opaque offsets, so every
    // load is issued unconditionally in scalar-base + VGPR-offset form.
    auto load_row = [&](int r, u4* ch) {
        const uint8_t* row = W + static_cast<int64_t>(r < M ? r : M - 1) * row_bytes;
#pragma unroll
        for (int c = 0; c < kChunkSlots; ++c) {
            const int cc = lane + kWave * c;
            uint32_t off = 16u * static_cast<uint32_t>(cc < nchunks ? cc : 0);
            asm volatile("" : "+v"(off));
            ch[c] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(row + off));
        }
    };
    // x passes through LDS once per workgroup (the row buffers, 4 * 34K/32
    // bytes, hold its 4K bytes), so each wave reads its quarters' x from LDS
    // instead of issuing its own strided global loads.  Aligned x: each lane
    // issues its float4 loads (up to kXSlots) before the first row's and
    // stores them once they arrive, so the row's loads stay in flight (gfx9
    // retires loads in issue order) and no lane waits for a load per store.
    float* xl = reinterpret_cast<float*>(row_lds);
    constexpr int kXSlots = 4;
    const bool xvec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (K >> 2) <= kXSlots * kGemvThreads;
    f4 xv[kXSlots];
    if (xvec) {  // workgroup-uniform
#pragma unroll
        for (int k = 0; k < kXSlots; ++k) {
            const int i = threadIdx.x + k * kGemvThreads;
            xv[k] = reinterpret_cast<const f4*>(x)[i < (K >> 2) ? i : 0];
        }
    }
    u4 ch[PF > 1 ? 2 : 1][kChunkSlots];
    if constexpr (PF > 0) load_row(wave, ch[0]);
    if constexpr (PF > 1) load_row(wave + nwaves, ch[1]);
    if (xvec) {
#pragma unroll
        for (int k = 0; k < kXSlots; ++k) {
            const int i = threadIdx.x + k * kGemvThreads;
            if (i < (K >> 2)) reinterpret_cast<f4*>(xl)[i] = xv[k];
        }
    } else if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        for (int i = threadIdx.x; i < (K >> 2); i += kGemvThreads)
            reinterpret_cast<f4*>(xl)[i] = reinterpret_cast<const f4*>(x)[i];
    } else {
        for (int i = threadIdx.x; i < K; i += kGemvThreads) xl[i] = x[i];
    }
    __syncthreads();
    float xs[SLOTS][8];
    bool on[SLOTS];
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int q = lane + kWave * s;
        on[s] = FULL || q < nq;
        const int qc = on[s] ? q : 0;  // a masked slot re-reads quarter 0: inside x
        const f4 a = reinterpret_cast<const f4*>(xl)[2 * qc];
        const f4 b = reinterpret_cast<const f4*>(xl)[2 * qc + 1];
        xs[s][0] = a.x; xs[s][1] = a.y; xs[s][2] = a.z; xs[s][3] = a.w;
        xs[s][4] = b.x; xs[s][5] = b.y; xs[s][6] = b.z; xs[s][7] = b.w;
        if constexpr (!FULL) {
#pragma unroll
            for (int j = 0; j < 8; ++j) xs[s][j] = on[s] ? xs[s][j] : 0.0f;
        }
    }
    __syncthreads();  // every wave has its x before any row overwrites the buffers

    auto row_step = [&](int r, u4* ch) {
        if constexpr (PF == 0) load_row(r, ch);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < kChunkSlots; ++c) {
            // a lane past the row's last chunk dumps its (clamped) chunk into
            // the pad, which nothing reads as data: no branch around the store
            const int cc = lane + kWave * c;
            uint8_t* dst = cc < nchunks ? buf + 16 * cc : pad;
            *reinterpret_cast<u4*>(dst) = ch[c];
        }
        if constexpr (PF > 0) {
            // the buffer's next row loads while this row is computed from LDS
            load_row(r + PF * nwaves, ch);
            __builtin_amdgcn_sched_barrier(0);
        }
        float acc = 0.0f;
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            // a masked slot re-reads block 0 of the row buffer; its product is discarded
            const uint32_t q_at = on[s] ? q_base0 + kSlotBytes * s : 0u;
            const uint32_t d_at = on[s] ? d_off0 + kSlotBytes * s : 0u;
            const uint32_t* w = reinterpret_cast<const uint32_t*>(buf + q_at);
            const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
            u2a2 qv;
            qv.x = __builtin_amdgcn_alignbyte(w1, w0, q_shift);
            qv.y = __builtin_amdgcn_alignbyte(w2, w1, q_shift);
            const uint16_t dv = *reinterpret_cast<const uint16_t*>(buf + d_at);
            const float bs = block_sum(q8_quarter_dot(qv, xs[s]));
            const float c = half_bits_to_float(dv) * bs;
            if constexpr (FULL) acc += c;
            else acc += on[s] ? c : 0.0f;
        }
        acc = wave_sum_of_quads(acc);
        // PF 2: every lane stores the (wave-uniform) sum, so no branch
        // separates the two buffers' loads and each wait stays exact
        if (PF > 1 || lane == 0) y[r] = acc;
    };
    if constexpr (PF < 2) {
        for (int r = wave; r < M; r += nwaves) row_step(r, ch[0]);
    } else {
        // rows in pairs with no branch between them, so each wait leaves the
        // other buffer's loads in flight; an odd last row after the loop
        int r = wave;
        for (; r + nwaves < M; r += 2 * nwaves) {
            row_step(r, ch[0]);
            row_step(r + nwaves, ch[1]);
        }
        if (r < M) row_step(r, ch[0]);
    }
}

// K > 8192: the same row walk with x re-read from L1/L2 per row.
__global__ __launch_bounds__(kGemvThreads) void gemv_q8_0_wide_kernel(float* __restrict__ y,
                                                                      const uint8_t* __restrict__ W,
                                                                      const float* __restrict__ x,
                                                                      int M, int K) {
    const int lane = threadIdx.x & (kWave - 1);
    const int nq = K >> 3;
    const int64_t row_bytes = static_cast<int64_t>(K >> 5) * 34;
    const int wave = static_cast<int>((blockIdx.x * static_cast<unsigned>(kGemvThreads) + threadIdx.x) / kWave);
    const int nwaves = static_cast<int>(gridDim.x * (kGemvThreads / kWave));
    for (int r = wave; r < M; r += nwaves) {
        const uint8_t* row = W + static_cast<int64_t>(r) * row_bytes;
        float acc = 0.0f;
        // nq is a multiple of 4, so a quad is either wholly inside or wholly past the row
        for (int q0 = 0; q0 < nq; q0 += kWave) {
            const int q = q0 + lane;
            const bool on = q < nq;
            const int qc = on ? q : 0;
            const int d_off = 34 * (qc >> 2);
            const u2a2 qv = __builtin_nontemporal_load(reinterpret_cast<const u2a2*>(row + d_off + 2 + 8 * (qc & 3)));
            const uint16_t dv = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(row + d_off));
            float xs[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) xs[j] = x[8 * qc + j];
            const float bs = block_sum(q8_quarter_dot(qv, xs));
            acc += (on && (lane & 3) == 0) ? half_bits_to_float(dv) * bs : 0.0f;
        }
        acc = wave_reduce(acc, OpAdd{});
        if (lane == 0) y[r] = acc;
    }
}

// K == 0: every row is an empty sum (the reference's loop body never runs).
__global__ __launch_bounds__(kGemvThreads) void gemv_q8_0_empty_kernel(float* __restrict__ y, int M) {
    const int r = static_cast<int>(blockIdx.x * kGemvThreads + threadIdx.x);
    if (r < M) y[r] = 0.0f;
}

// The staged kernel's workgroups per CU: 4, below the occupancy limit (7 per
// CU at K = 2560).  Of caps 2-8 on the two LM-head shapes, 4 is the best at
// 151936 x 2560 (63-64 us against 66-67 at the limit, 70-72 at 2 or 3) and
// level with the limit at 128256 x 4096 (89-92 us); 3 there ran 86-87 us in
// a process of its own but 93-96 after the rest of a benchmark run.
constexpr int q8_staged_wg_per_cu(int K) {
#ifdef FENCE_GEMV_Q8_WG_PER_CU
    return static_cast<void>(K), FENCE_GEMV_Q8_WG_PER_CU;
#else
    return static_cast<void>(K), 4;
#endif
}

// Workgroups that fit on the device at once for `kernel` with `lds` bytes of
// dynamic LDS, at most `cap` per CU.  The occupancy query is cached per
// (kernel, device): a template instance's static is one per kernel.
template <class Kernel>
int resident_grid(Kernel kernel, size_t lds, int cap, unsigned* grid) {
    static std::atomic<int> cache[64];
    static std::atomic<int> cache_cus[64];
    static std::atomic<size_t> cache_lds[64];
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_status(e);
    if (dev < 0 || dev >= 64) return FENCE_ERROR_INVALID_VALUE;
    int per_cu = cache[dev].load(std::memory_order_acquire);
    int cus = cache_cus[dev].load(std::memory_order_relaxed);
    if (per_cu == 0 || cus == 0 || cache_lds[dev].load(std::memory_order_relaxed) != lds) {
        if (hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev); e != hipSuccess)
            return hip_status(e);
        if (hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kGemvThreads, lds);
            e != hipSuccess)
            return hip_status(e);
        if (per_cu < 1) per_cu = 1;
        if (cus < 1) cus = 1;
        cache_lds[dev].store(lds, std::memory_order_relaxed);
        cache_cus[dev].store(cus, std::memory_order_relaxed);
        cache[dev].store(per_cu, std::memory_order_release);
    }
    // a grid read against another lds's entry is still a valid grid (every
    // kernel strides over its rows); only its size would be off
    *grid = static_cast<unsigned>(cus * (per_cu < cap ? per_cu : cap));
    return FENCE_SUCCESS;
}

template <class Kernel>
int launch_rows(Kernel kernel, float* y, const uint8_t* W, const float* x, int M, int K, int rows_per_wave,
                size_t lds, hipStream_t s, int cap = 8) {
    unsigned grid = 0;
    if (int st = resident_grid(kernel, lds, cap, &grid); st != FENCE_SUCCESS) return st;
    const int64_t per_wg = static_cast<int64_t>(kGemvThreads / kWave) * rows_per_wave;
    const int64_t wanted = (M + per_wg - 1) / per_wg;
    if (wanted < grid) grid = static_cast<unsigned>(wanted);
    return launch(kernel, dim3(grid), dim3(kGemvThreads), lds, s, y, W, x, M, K);
}

template <int SLOTS>
int launch_slots(float* y, const uint8_t* W, const float* x, int M, int K, hipStream_t s) {
    const bool full = K == kWave * 8 * SLOTS;
    if (FENCE_GEMV_Q8_STAGED && K % 256 == 0 && aligned(W, 16)) {
        const size_t lds = static_cast<size_t>(kGemvThreads / kWave) * (K / 32) * 34 + 16;
        constexpr int pf = FENCE_GEMV_Q8_PREFETCH;
        const int cap = q8_staged_wg_per_cu(K);
        if (full) return launch_rows(gemv_q8_0_staged_kernel<SLOTS, true, pf>, y, W, x, M, K, 1, lds, s, cap);
        return launch_rows(gemv_q8_0_staged_kernel<SLOTS, false, pf>, y, W, x, M, K, 1, lds, s, cap);
    }
    if (full)
        return launch_rows(gemv_q8_0_kernel<SLOTS, FENCE_GEMV_Q8_ROWS, true>, y, W, x, M, K, FENCE_GEMV_Q8_ROWS, 0, s);
    return launch_rows(gemv_q8_0_kernel<SLOTS, FENCE_GEMV_Q8_ROWS, false>, y, W, x, M, K, FENCE_GEMV_Q8_ROWS, 0, s);
}

int gemv_q8_0_launch(float* y, const void* Wv, const float* x, int M, int K, hipStream_t s) {
    if (M < 0 || K < 0 || (K % 32) != 0) return FENCE_ERROR_INVALID_VALUE;
    if (M == 0) return FENCE_SUCCESS;
    if (!y || !Wv || (K > 0 && !x)) return FENCE_ERROR_INVALID_VALUE;
    const uint8_t* W = static_cast<const uint8_t*>(Wv);
    if (!aligned(W, 2)) return FENCE_ERROR_INVALID_VALUE;  // block_q8_0 holds an fp16: 2-byte aligned by type
    if (K == 0)
        return launch(gemv_q8_0_empty_kernel, dim3(grid_1d(M, kGemvThreads)), dim3(kGemvThreads), 0, s, y, M);
    const int slots = (K / 8 + kWave - 1) / kWave;
    switch (slots) {
        case 1: return launch_slots<1>(y, W, x, M, K, s);
        case 2: return launch_slots<2>(y, W, x, M, K, s);
        case 3: return launch_slots<3>(y, W, x, M, K, s);
        case 4: return launch_slots<4>(y, W, x, M, K, s);
        case 5: return launch_slots<5>(y, W, x, M, K, s);
        case 6: return launch_slots<6>(y, W, x, M, K, s);
        case 7:
        case 8: return launch_slots<8>(y, W, x, M, K, s);
        case 9:
        case 10: return launch_slots<10>(y, W, x, M, K, s);
        case 11:
        case 12: return launch_slots<12>(y, W, x, M, K, s);
        case 13:
        case 14:
        case 15:
        case 16: return launch_slots<16>(y, W, x, M, K, s);
        default: return launch_rows(gemv_q8_0_wide_kernel, y, W, x, M, K, 1, 0, s);
    }
}

}  // namespace
}  // namespace fence

extern "C" int fence_gemv_q8_0(const void* W, const float* x, float* y, int M, int K, hipStream_t stream) {
    return fence::gemv_q8_0_launch(y, W, x, M, K, stream);
}
