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
// Every kernel adds a row's terms in one order that depends on K alone
// (q6_wpr, q6_passes), so a row has the same bits in every launch.
#include <atomic>
#include <type_traits>

#include "common.hpp"

// How a row's blocks are split over waves (see q6_wpr): 0 up to four passes
// (16 blocks) per wave, 1 up to two, 2 one pass where the row allows.
#ifndef FENCE_GEMV_Q6K_SPLIT
#define FENCE_GEMV_Q6K_SPLIT 0
#endif
// 1: an occupancy-sized grid of workgroups looping over row groups;
// 0: one workgroup per row group.
#ifndef FENCE_GEMV_Q6K_RESIDENT
#define FENCE_GEMV_Q6K_RESIDENT 1
#endif
// 1: the resident grid is trimmed so every workgroup gets the same number of
// row groups: with G groups and room for W workgroups, ceil(G / W) rounds
// need only ceil(G / rounds) workgroups.  0 (kept): W workgroups, the last
// round partly empty.  Results do not depend on the grid.  Measured on
// MI355X, Qwen3-4B decode steps (bench.py --decode-only, 64 tokens, two
// interleaved runs each): 1,852 and 1,854 us per token with 1 against 1,768
// and 1,767 with 0 -- wave lifetimes vary by several us within a launch
// whatever the group count, so fewer workgroups only lose parallelism.
// Most workgroups per CU in a resident grid (0: as many as fit).  6 trims
// the 4-wave launches (down: 7 fit, o: 8) and leaves the 8-wave ones (2
// fit); decode steps ran ~10 us per token faster than with every resident
// workgroup, and slower with 5 (+15-20 us) or level with 4.
#ifndef FENCE_GEMV_Q6K_WG_PER_CU
#define FENCE_GEMV_Q6K_WG_PER_CU 6
#endif
#ifndef FENCE_GEMV_Q6K_BALANCED
#define FENCE_GEMV_Q6K_BALANCED 0
#endif
// 1: rows of 33-40 blocks take two waves of up to five passes (20 block
// slots for 17-20 blocks) instead of four waves of three passes (12 slots for
// 8-10 blocks, the rest masked); 0 (kept): four waves.  The wider form issues
// 22% fewer loop instructions per row but needs 111 VGPRs (4 waves per SIMD
// against 7): Qwen3-4B decode steps 1,722-1,724 us per token against 1,713
// (bench.py --decode-only against a `make TAG=nowide
// EXTRA=-DFENCE_GEMV_Q6K_WIDE=0` build, interleaved runs on one box).
#ifndef FENCE_GEMV_Q6K_WIDE
#define FENCE_GEMV_Q6K_WIDE 0
#endif
// Launches of at most this many rows of 13-16 blocks take the one-wave layout
// spread over four waves per row (XW below; same results, bit for bit).
// Measured on MI355X, p50: the 2560 x 4096 o projection runs in 4.96 us with
// four waves per row, 5.36 with two (two passes each, so every row of it fits
// the GPU at once) and 6.00 with one.
#ifndef FENCE_GEMV_Q6K_XW_ROWS
#define FENCE_GEMV_Q6K_XW_ROWS 8192
#endif

// Gate/up pairs of rows of at most 16 blocks: 0 the staged pair kernel (a
// row's gate and up on different waves); 4 or 8 the kernel with one wave per
// output row (gemv_q6k_pairw_kernel), that many waves per workgroup.  Results
// are the same bits either way.  Measured on MI355X, Qwen3-4B decode steps
// (bench.py --decode-only, 64 tokens, two interleaved runs of each build):
// 0: 1,710-1,713 us per token; 8 with the prefetch (kept): 1,683-1,684, and
// 1,691-1,694 without it; 4: 1,688-1,691, and 1,704-1,707 without it.
#ifndef FENCE_GEMV_Q6K_PAIRW
#define FENCE_GEMV_Q6K_PAIRW 8
#endif
static_assert(FENCE_GEMV_Q6K_PAIRW == 0 || FENCE_GEMV_Q6K_PAIRW == 4 || FENCE_GEMV_Q6K_PAIRW == 5 ||
                  FENCE_GEMV_Q6K_PAIRW == 8 || FENCE_GEMV_Q6K_PAIRW == 10,
              "FENCE_GEMV_Q6K_PAIRW: 0, 4, 5, 8 or 10");
// Waves per SIMD the one-wave pair kernel's registers are fitted to: 4 (104
// VGPRs) or 5 (93, no spills).  More resident waves run slower: decode steps
// (as above) 1,682 us per token at 4 against 1,685-1,687 at 5 with 8-wave
// workgroups (two per CU either way), 1,719-1,721 with 4-wave workgroups (20
// waves per CU), 1,762-1,764 with 5-wave and 1,806-1,808 with 10-wave ones.
#ifndef FENCE_GEMV_Q6K_PAIRW_WPE
#define FENCE_GEMV_Q6K_PAIRW_WPE 4
#endif
// 1: rows whose last pass holds two blocks (nb % 4 == 2) share that pass
// between gate and up in the one-wave pair kernel (MERGE there); 0: each row
// its own.  Same results, bit for bit.
#ifndef FENCE_GEMV_Q6K_PAIRW_MERGE
#define FENCE_GEMV_Q6K_PAIRW_MERGE 1
#endif
// 1: the one-wave pair kernel loads the next output row while the current
// one is computed; 0: each row after the previous one.
#ifndef FENCE_GEMV_Q6K_PAIRW_PF
#define FENCE_GEMV_Q6K_PAIRW_PF 1
#endif

// 1: the staged kernel loads a wave's next row group while the current one is
// computed (as XW launches do) in the one-wave launches with the RMSNorm
// prologue (q/k/v) -- PF_NORM -- and in launches of several waves per row
// (down) -- PF_SPLIT; 0: each group after the previous one.  Same results.
// Measured as above: 1,693 us per token with PF_NORM against 1,685-1,687
// without (97 VGPRs: 4 waves per SIMD instead of 5), 1,681-1,682 with
// PF_SPLIT (within the spread of the session's runs).
#ifndef FENCE_GEMV_Q6K_PF_NORM
#define FENCE_GEMV_Q6K_PF_NORM 0
#endif
#ifndef FENCE_GEMV_Q6K_PF_SPLIT
#define FENCE_GEMV_Q6K_PF_SPLIT 0
#endif

// 1: every wave of the staged kernel records its entry and exit times on the
// device's constant wall clock (100 MHz), its hardware placement and its
// row-group count into `wave_clock` (read back by fence_wave_clock_read).
// Only the instrumented library (libfence_ops_waveclock.so) is built with it;
// the product library is not, and its kernels are unchanged.
#ifndef FENCE_WAVE_CLOCK
#define FENCE_WAVE_CLOCK 0
#endif

namespace fence {
namespace {

constexpr int kThreads = 256;

#if FENCE_WAVE_CLOCK
// One record of four words per wave of a launch (the last launch's):
// entry time, exit time, HW_ID | XCC_ID << 32, row groups computed.
constexpr int kWaveClockMax = 1 << 16;
static __device__ __align__(256) uint64_t wave_clock[4 * kWaveClockMax];
#endif

// Wave entry and exit for FENCE_WAVE_CLOCK builds (empty otherwise).  Each
// writes its words straight away (lane 0, vector stores) and keeps nothing
// live across the kernel, to leave the kernel's register allocation as it is.
[[maybe_unused]] __device__ __forceinline__ void wave_clock_enter(int64_t wave, int lane) {
#if FENCE_WAVE_CLOCK
    const uint64_t t = __builtin_amdgcn_s_memrealtime();
    if (lane == 0 && wave < kWaveClockMax) wave_clock[4 * wave] = t;
#else
    (void)wave;
    (void)lane;
#endif
}

// groups: the row groups (or rows) the wave computed
[[maybe_unused]] __device__ __forceinline__ void wave_clock_leave_n(int64_t wave, int lane, int64_t groups) {
#if FENCE_WAVE_CLOCK
    const uint64_t t = __builtin_amdgcn_s_memrealtime();
    // HW_ID (hardware register 4) and XCC_ID (20), all 32 bits of each
    const uint32_t hw = __builtin_amdgcn_s_getreg(4 | (31 << 11));
    const uint32_t xcc = __builtin_amdgcn_s_getreg(20 | (31 << 11));
    if (lane == 0 && wave < kWaveClockMax) {
        uint64_t* r = wave_clock + 4 * wave;
        r[1] = t;
        r[2] = static_cast<uint64_t>(hw) | (static_cast<uint64_t>(xcc) << 32);
        r[3] = static_cast<uint64_t>(groups);
    }
#else
    (void)wave;
    (void)lane;
    (void)groups;
#endif
}

// groups: the wave's row groups g = blockIdx.x + k * gridDim.x < n_groups
[[maybe_unused]] __device__ __forceinline__ void wave_clock_leave(int64_t wave, int lane, int64_t n_groups) {
    const int64_t groups = n_groups > blockIdx.x ? (n_groups - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;
    wave_clock_leave_n(wave, lane, groups);
}
constexpr int kBlockBytes = 210;
constexpr int kMaxSegBlocks = 16;  // blocks of one row staged by one wave

// The 16 quants (0..63) of one lane of one block, one byte each: w[c] holds
// column c's four (l = 4j .. 4j+3).
struct Q6Lane {
    uint32_t w[4];
};

// Every byte of c holds column 0's high bits in bits 0-1, column 1's in
// 2-3, column 2's in 4-5 and column 3's in 6-7.  ce keeps columns 0 and 2
// (bits 0-1, 4-5), co columns 1 and 3 moved to the same places; each
// column's byte is then one bit-field insert, (nibble & 0x0F) | (bits above
// 0x0F of the crumb word), whose bits 6-7 are clear.  Written as asm: the
// compiler folds the masks back into its own three-operation form.
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t x, uint32_t y) {  // (x & m) | (y & ~m)
    uint32_t r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(m), "v"(x), "v"(y));
    return r;
}

__device__ __forceinline__ Q6Lane q6_unpack(uint32_t a, uint32_t b, uint32_t c) {
    constexpr uint32_t kNib = 0x0F0F0F0Fu;  // low nibble of every byte
    constexpr uint32_t kTwo = 0x33333333u;  // bits 0-1 and 4-5 of every byte
    const uint32_t ce = c & kTwo;
    const uint32_t co = (c >> 2) & kTwo;
    Q6Lane r;
    r.w[0] = bfi(kNib, a, ce << 4);
    r.w[1] = bfi(kNib, b, co << 4);
    r.w[2] = bfi(kNib, a >> 4, ce);
    r.w[3] = bfi(kNib, b >> 4, co);
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
// fp32 rounding of terms of size 1056 |x|.  Two v_dot2_f32_f16 against
// (-1056, -1056), which binary16 holds exactly (every product is exact in
// fp32): 2 operations per column where converting and adding the four x
// takes 8.
__device__ __forceinline__ float q6_col_bias(uint32_t x01, uint32_t x23) {
    const h2 k = {static_cast<_Float16>(-1056.0f), static_cast<_Float16>(-1056.0f)};
    const float t = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, x01), k, 0.0f, false);
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, x23), k, t, false);
}

// d * sum_c sc_c * sum_k (q - 32) * x over the lane's 16 weights of one block,
// each pair of weights one v_dot2c_f32_f16.  Contraction off: the product
// d * acc is rounded on its own and never fused into the caller's sum, so
// every kernel layout that adds the same lane values in the same order gets
// the same bits.
// a . b + c in the three-operand v_dot2_f32_f16.  The builtin's form is
// shrunk to the two-operand v_dot2c_f32_f16 (d += a . b) wherever it can be,
// which for a chain starting from a loop-invariant c costs a v_mov copy of c
// first; this keeps c where it is.  Same instruction arithmetic, same bits.
__device__ __forceinline__ float dot2_f16(h2 a, h2 b, float c) {
    float d;
    asm("v_dot2_f32_f16 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}

// d * acc is one v_fma_mix_f32 with the binary16 d as its operand and 0
// added: the product's value, rounded once, except that a zero product is
// +0 whatever its sign (the lane values are only added, and a +0 in place
// of a -0 changes no nonzero sum).
__device__ __forceinline__ float q6_lane_dot(const Q6Lane& q, const uint32_t* xh, const float* kb, const int* sc,
                                             _Float16 d) {
#pragma clang fp contract(off)
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        float p = dot2_f16(q6_pair(q.w[c], 0x00050004u), __builtin_bit_cast(h2, xh[2 * c]), kb[c]);
        p = __builtin_amdgcn_fdot2(q6_pair(q.w[c], 0x00070006u), __builtin_bit_cast(h2, xh[2 * c + 1]), p, false);
        acc = __builtin_fmaf(static_cast<float>(sc[c]), p, acc);
    }
    float r;
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(d), "v"(acc));
    return r;
}

__device__ __forceinline__ float wave_sum(float v) { return wave_reduce(v, OpAdd{}); }

// The segment [b0, b1) of the row's blocks a wave handles when WPR waves
// share a row: an even split.
__device__ __forceinline__ void segment(int nb, int seg, int wpr, int* b0, int* b1) {
    *b0 = (nb * seg) / wpr;
    *b1 = (nb * (seg + 1)) / wpr;
}

// The order a row of nb blocks is summed in, for every kernel: WPR waves (or
// segments) per row, each over PASSES passes of four blocks; each segment's
// lane values are added in pass order (a masked block slot adds +0), summed
// over the wave, and the segment sums added in segment order.  It depends on
// nb alone, so a row gets the same bits from every launch that contains it:
// alone or with other matrices, staged or direct.  Rows of more than 64
// blocks are never staged; the direct kernel gives them one segment.
__host__ __device__ constexpr int q6_wpr(int nb) {
    return nb > 4 * kMaxSegBlocks        ? 1
           : FENCE_GEMV_Q6K_SPLIT == 2 ? (nb <= 4 ? 1 : nb <= 8 ? 2 : 4)
           : FENCE_GEMV_Q6K_SPLIT == 1 ? (nb <= 8 ? 1 : nb <= 16 ? 2 : 4)
                                       : (nb <= 16 ? 1 : nb <= (FENCE_GEMV_Q6K_WIDE ? 40 : 32) ? 2 : 4);
}
__host__ __device__ constexpr int q6_passes(int nb) { return (nb + 4 * q6_wpr(nb) - 1) / (4 * q6_wpr(nb)); }

// The lane's x pairs of every pass (binary16 zeros for a masked block).
// Loads only: load_x_bias then forms the column biases, so loads issued in
// between stay in flight while the biases wait for x.
template <int PASSES>
__device__ __forceinline__ void load_x_pairs(uint32_t (&xh)[PASSES][8], const uint16_t* x16, int b0, int b1,
                                             int bslot, int h, int j) {
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
        }
    }
}

template <int PASSES>
__device__ __forceinline__ void load_x_bias(const uint32_t (&xh)[PASSES][8], float (&kb)[PASSES][4]) {
#pragma unroll
    for (int p = 0; p < PASSES; ++p)
#pragma unroll
        for (int c = 0; c < 4; ++c) kb[p][c] = q6_col_bias(xh[p][2 * c], xh[p][2 * c + 1]);
}

template <int PASSES>
__device__ __forceinline__ void load_x(uint32_t (&xh)[PASSES][8], float (&kb)[PASSES][4], const uint16_t* x16,
                                       int b0, int b1, int bslot, int h, int j) {
    load_x_pairs<PASSES>(xh, x16, b0, b1, bslot, h, j);
    load_x_bias<PASSES>(xh, kb);
}

// A launch's matrices: up to kMaxMats row blocks that share x and K, their
// rows numbered one after another (matrix i holds rows [end[i-1], end[i])).
// PAIR: two matrices of M rows each, gate and up, combined per row into
// act = silu(gate x) * (up x), written as binary16 (act16) and optionally
// fp32 (act32) -- src/model/qwen3.cu:328-336 in one pass.
constexpr int kMaxMats = 4;
struct Q6Job {
    const uint8_t* W[kMaxMats];
    float* y[kMaxMats];
    const float* bias[kMaxMats];
    int end[kMaxMats];
    int n;
    uint16_t* act16;
    float* act32;
};

// NORM launches: x is the layer-boundary row (src/model/qwen3.cu:267-275 and
// :310-325), h = hid + res (hid alone when res is null) and
// x = binary16(rms_norm(h) * w), which every workgroup computes in its
// prologue.  The sum of squares follows the row RMSNorm kernel (rms_norm.hip)
// at its launch shape for the row, T threads and vpt (1 or 2) float4s per
// lane: lane f's partial is dot4(float4 f) + dot4(float4 f + T), each 64
// consecutive lanes reduce as one wave, and the T / 64 wave sums are added
// in order -- so x is bit-identical to that kernel's.  Workgroup 0 also
// writes h to hid_out (with res) and x to x_out.
struct RmsIn {
    const float* hid;
    const float* res;
    float* hid_out;
    const float* w;
    uint16_t* x_out;
    float eps;
    int T;
    int vpt;
};

// Matrix of global row r (wave-uniform), and r's row within it.
__device__ __forceinline__ int mat_of(const Q6Job& job, int64_t r, int64_t* lr) {
    int m = 0;
#pragma unroll
    for (int k = 0; k < kMaxMats - 1; ++k) m += (k < job.n - 1 && r >= job.end[k]) ? 1 : 0;
    *lr = r - (m ? job.end[m - 1] : 0);
    return m;
}

// Waves of a staged workgroup: 4; 8 for a gate/up pair whose rows take four
// waves each; 8 for a launch that normalises its input row in the prologue
// with one wave per row (every workgroup computes the row norm, so wider
// workgroups compute it fewer times per CU).  Measured on MI355X: two 8-wave
// workgroups per CU instead of five 4-wave ones cut q/k/v from 9.04 to
// 7.28 us (K = 2560) and from 10.44 to 9.40 us (K = 4096), p50; 6-, 10- and
// 12-wave workgroups were slower (a workgroup's waves spread over the CU's
// four SIMDs, so only multiples of four fill it).  The gate/up pair with its
// norm runs at 6 waves per SIMD (80 VGPRs), three 8-wave workgroups per CU:
// Qwen3-4B decode steps 1,718 -> 1,710 us per token against six 4-wave ones
// (bench.py --decode-only, interleaved runs).  A row's arithmetic does not
// depend on the workgroup, so every result is the same.
template <int WPR, bool PAIR, int NORM = 0>
constexpr int staged_waves() { return NORM && WPR == 1 ? 8 : (PAIR && WPR == 4 ? 8 : 4); }

// Staged kernel.  WPR waves per row (1, 2 or 4), each over at most 4 * PASSES
// <= 16 blocks.  LDS: one buffer of kSegBytes per wave + red[].  A workgroup
// of NW waves takes NW / WPR rows per group; with PAIR the first half of them
// are gate rows and the second half the same rows of up.  NORM: x from
// `rin` (see RmsIn), staged through the same LDS before the first group's
// blocks are; NORM (1 or 2) is the norm kernel's float4s per lane, rin.vpt.
// XW (PASSES * WPR = 4, rows of 13-16 blocks): the one-wave layout <4, 1>
// spread over WPR waves -- wave s takes passes PASSES*s .. PASSES*s +
// PASSES - 1 (blocks from 4 * PASSES * s on), and each pass's lane values go
// to LDS, where the row's first wave adds each lane's four in pass order
// before the wave sum: the additions of one wave doing four passes, so the
// rows are bit-identical to <4, 1>'s, computed by WPR times as many waves.
// XW launches also load each wave's next row group while the current one is
// computed (one chunk slot per lane: 4 VGPRs).  Measured on MI355X, p50 of
// 400, in-process A/B: the o projection 2560 x 4096 4.92 -> 4.60 us, Llama-3-8B
// 4096 x 4096 6.44 -> 5.80 us; the same prefetch in the other layouts cost
// more registers than it saved (gate/up pair, 9728 x 2560) or changed nothing.
// VW (NORM launches): the norm's 64-lane virtual waves each wave holds,
// ceil((T / 64) / NW), chosen at launch so no slot is always empty (a slot
// costs its loads, masks and reductions whether or not it is used).
// CLOCK: the instrumented copy (FENCE_WAVE_CLOCK builds launch it on the grid
// the plain kernel gets); every product launch has CLOCK = false.
template <int PASSES, int WPR, bool PAIR, bool MULTI, int NORM, bool XW = false, bool CLOCK = false, int VW = 0>
__global__ __launch_bounds__((kWave * staged_waves<WPR, PAIR, NORM>())) void gemv_q6k_staged_kernel(
    const Q6Job job, const uint16_t* __restrict__ x16, int nb, const RmsIn rin) {
    static_assert(!XW || (PASSES * WPR == 4 && !PAIR && NORM == 0), "XW: four passes, plain rows");
    // prefetch the next row group: XW launches, and where the switches below ask
    constexpr bool PF = XW || (FENCE_GEMV_Q6K_PF_NORM && NORM != 0 && WPR == 1 && !PAIR) ||
                        (FENCE_GEMV_Q6K_PF_SPLIT && NORM == 0 && WPR > 1 && !PAIR);
    constexpr int NW = staged_waves<WPR, PAIR, NORM>();
    constexpr int kSegBytes = 4 * PASSES * kBlockBytes + 32;  // + alignment slack
    constexpr int kBufBytes = (kSegBytes + 15) / 16 * 16;
    constexpr int kChunkSlots = (kSegBytes / 16 + kWave - 1) / kWave;
    constexpr int kRowsPerGroup = NW / WPR;
    constexpr int kOutPerGroup = PAIR ? kRowsPerGroup / 2 : kRowsPerGroup;
    static_assert(!PAIR || kRowsPerGroup >= 2, "a pair needs two rows per group");
    constexpr uint32_t kPassBytes = 4 * kBlockBytes;  // 840: a multiple of 4
    // NORM: binary16 x of the longest row this shape takes (nb <= 4 * PASSES * WPR)
    constexpr int kStageBytes = NW * kBufBytes;
    constexpr int kNormXBytes = 2 * 1024 * PASSES * WPR;
    constexpr int kLdsBytes = NORM && kNormXBytes > kStageBytes ? kNormXBytes : kStageBytes;
    __shared__ __align__(16) uint8_t lds[kLdsBytes];
    __shared__ float red[NW];
    __shared__ float nred[NORM ? 16 : 1];  // the row norm's wave sums (T <= 1024)
    __shared__ float xr[XW ? NW : 1][XW ? PASSES : 1][kWave];  // XW: each pass's lane values
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));  // wave-uniform
    if constexpr (CLOCK) wave_clock_enter(static_cast<int64_t>(blockIdx.x) * NW + wid, lane);
    const int seg = wid % WPR;
    const int rslot = wid / WPR;
    uint8_t* buf = lds + wid * kBufBytes;
    const int bslot = lane >> 4, h = (lane >> 3) & 1, j = lane & 7;
    int b0, b1;
    if constexpr (XW) {
        b0 = 4 * PASSES * seg;  // nb > 12: every wave has at least one block
        b1 = b0 + 4 * PASSES < nb ? b0 + 4 * PASSES : nb;
    } else {
        segment(nb, seg, WPR, &b0, &b1);
    }
    const int64_t row_bytes = static_cast<int64_t>(nb) * kBlockBytes;
    const int64_t n_out = PAIR ? job.end[0] : job.end[job.n - 1];  // rows (PAIR: output rows)

    uint32_t xh[PASSES][8];
    float kb[PASSES][4];
    if constexpr (!NORM) load_x_pairs<PASSES>(xh, x16, b0, b1, bslot, h, j);  // biases once the first group is out

    // NORM, first half: the row's loads, issued before the first group's
    // blocks.  Wave w holds the row norm's waves w, w + NW, ... (vw < T / 64);
    // a slot past the row holds zeros, as in the norm kernel.
    // Every load is unconditional (clamped slots, and hidden again in place of
    // an absent residual), so all are in flight together and none waits for
    // the blocks issued after them.
    static_assert(NORM == 0 || (VW >= 1 && VW * NW <= 16 + NW - 1), "VW: 1 .. ceil(16 / NW) slots");
    constexpr int kVW = NORM ? VW : 1;
    constexpr int kVpt = NORM ? NORM : 1;
    f4 nh[kVW][kVpt], nr[kVW][kVpt], nw[kVW][kVpt];
    auto norm_slot = [&](int i, int jj, int* f) {
        const int vw = wid + NW * i;
        *f = vw * kWave + lane + jj * rin.T;
        return vw * kWave < rin.T && *f < nb * 64;
    };
    if constexpr (NORM != 0) {
        const float* rp = rin.res ? rin.res : rin.hid;
#pragma unroll
        for (int i = 0; i < kVW; ++i) {
#pragma unroll
            for (int jj = 0; jj < kVpt; ++jj) {
                int f;
                const int fc = norm_slot(i, jj, &f) ? f : 0;
                nh[i][jj] = ld4<false>(rin.hid + 4 * fc);
                nr[i][jj] = ld4<false>(rp + 4 * fc);
                nw[i][jj] = ld4<false>(rin.w + 4 * fc);
            }
        }
    }
    bool on[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) on[p] = b0 + 4 * p + bslot < b1;
    const uint32_t lane_ql = 64 * h + 4 * j;         // ql dword of the lane in its block
    const uint32_t lane_qh = 128 + 32 * h + 4 * j;   // qh dword
    const uint32_t lane_sc = 192 + 8 * h + (j >> 2);  // column 0's scale byte
    const uint32_t blk_off = static_cast<uint32_t>(bslot) * kBlockBytes;

    // The row this wave computes in group g: its output index o (a global row
    // without PAIR), matrix m and row lr within the matrix; o >= n_out past the end.
    auto row_of = [&](int64_t g, int64_t* o, int* m, int64_t* lr) {
        if constexpr (PAIR) {
            *o = g * kOutPerGroup + rslot % kOutPerGroup;
            *m = rslot / kOutPerGroup;
            *lr = *o < n_out ? *o : n_out - 1;  // clamped: loads past the end stay inside W
        } else if constexpr (MULTI) {
            *o = g * kRowsPerGroup + rslot;
            *m = mat_of(job, *o < n_out ? *o : n_out - 1, lr);
        } else {
            *o = g * kRowsPerGroup + rslot;
            *m = 0;
            *lr = *o < n_out ? *o : n_out - 1;
        }
    };
    // The 16-byte chunks covering the segment: [a0, a0 + 16 * nch) of job.W[m].
    auto seg_of = [&](int64_t lr, int64_t* a0, int* nch, uint32_t* delta) {
        const int64_t start = lr * row_bytes + static_cast<int64_t>(b0) * kBlockBytes;
        const int64_t end = lr * row_bytes + static_cast<int64_t>(b1) * kBlockBytes;
        *a0 = start & ~int64_t(15);
        *nch = static_cast<int>((end - *a0 + 15) >> 4);
        *delta = static_cast<uint32_t>(start - *a0);
    };
    // Loads of one segment's chunks: clamped and opaque offsets, so every
    // load is issued unconditionally in scalar-base + VGPR-offset form.
    auto load_seg = [&](const uint8_t* Wm, int64_t a0, int nch, u4* ch) {
        const uint8_t* src = Wm + a0;
#pragma unroll
        for (int k = 0; k < kChunkSlots; ++k) {
            const int cc = lane + kWave * k;
            uint32_t off = 16u * static_cast<uint32_t>(cc < nch ? cc : 0);
            asm volatile("" : "+v"(off));
            ch[k] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(src + off));
        }
    };
    u4 ch[kChunkSlots];
    if constexpr (NORM != 0) {
        // Second half, while the first group's blocks are in flight (the loop
        // below does not load them again): the norm kernel's reduction, x into
        // LDS, then each lane's x values.
        {
            int64_t o, lr, a0;
            int m, nch;
            uint32_t delta;
            row_of(blockIdx.x, &o, &m, &lr);
            seg_of(lr, &a0, &nch, &delta);
            load_seg(job.W[m], a0, nch, ch);
        }
        // h = hid (+ res), zero past the row; workgroup 0 stores it; then
        // each slot keeps only w * h, the first product of the norm's output
        const int nvw = rin.T / kWave;
        const bool has_res = rin.res != nullptr;
#pragma unroll
        for (int i = 0; i < kVW; ++i) {
#pragma unroll
            for (int jj = 0; jj < kVpt; ++jj) {
                int f;
                const bool ok = norm_slot(i, jj, &f);
                const f4 hv = has_res ? nh[i][jj] + nr[i][jj] : nh[i][jj];
                nh[i][jj] = ok ? hv : f4(0.0f);
                if (blockIdx.x == 0 && has_res && ok) st4<false>(rin.hid_out + 4 * f, hv);
            }
        }
#pragma unroll
        for (int i = 0; i < kVW; ++i) {
            const int vw = wid + NW * i;
            if (vw < nvw) {  // wave-uniform
                // the norm kernel's partial: its loop over two float4 slots
                float ss = 0.0f;
                ss += dot4(nh[i][0]);
                ss += kVpt > 1 ? dot4(nh[i][kVpt - 1]) : 0.0f;
                ss = wave_reduce(ss, OpAdd{});
                if (lane == 0) nred[vw] = ss;
            }
        }
#pragma unroll
        for (int i = 0; i < kVW; ++i)
#pragma unroll
            for (int jj = 0; jj < kVpt; ++jj) nw[i][jj] = nw[i][jj] * nh[i][jj];
        __syncthreads();
        float tot = nred[0];
        for (int v = 1; v < nvw; ++v) tot += nred[v];
        const float rs = rsqrtf(tot / static_cast<float>(nb * 256) + rin.eps);
        uint16_t* xs = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
        for (int i = 0; i < kVW; ++i) {
#pragma unroll
            for (int jj = 0; jj < kVpt; ++jj) {
                int f;
                if (norm_slot(i, jj, &f)) {
                    const f4 o = nw[i][jj] * rs;  // (w * h) * rs
                    st_h4<false>(xs + 4 * f, o);
                    if (blockIdx.x == 0) st_h4<false>(rin.x_out + 4 * f, o);
                }
            }
        }
        __syncthreads();
        load_x<PASSES>(xh, kb, xs, b0, b1, bslot, h, j);
        __syncthreads();  // lds holds staged blocks from here on
    }
    // One row group; LOADED: its blocks are already in ch (the NORM
    // prologue's first group), so the loop itself loads unconditionally.
    auto run_group = [&](int64_t g, auto loaded) {
        int64_t o, lr;
        int m;
        row_of(g, &o, &m, &lr);
        const bool valid = o < n_out;  // wave-uniform
        float part = 0.0f;
        int64_t a0;
        int nch;
        uint32_t delta;
        seg_of(lr, &a0, &nch, &delta);
        if constexpr (!decltype(loaded)::value) load_seg(job.W[m], a0, nch, ch);
        if (valid) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < kChunkSlots; ++k) {
                const int cc = lane + kWave * k;
                // a lane past the segment's last chunk stores into the slack
                // at the buffer's end, which holds no block data
                const uint32_t dst = cc < nch ? 16u * cc : static_cast<uint32_t>(kBufBytes - 16);
                *reinterpret_cast<u4*>(buf + dst) = ch[k];
            }
            if constexpr (PF) {  // the next group's chunks, in flight during this group's dot products
                const int64_t gn = g + gridDim.x;
                if (gn * kOutPerGroup < n_out) {  // workgroup-uniform
                    int64_t on, lrn, an;
                    int mn, ncn;
                    uint32_t dn;
                    row_of(gn, &on, &mn, &lrn);
                    seg_of(lrn, &an, &ncn, &dn);
                    load_seg(job.W[mn], an, ncn, ch);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        if (valid) {
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
                const _Float16 d = __builtin_bit_cast(_Float16, dbits);
                const float v = q6_lane_dot(q6_unpack(a, bq, c), xh[p], kb[p], sc, d);
                if constexpr (XW) xr[wid][p][lane] = on[p] ? v : 0.0f;
                else part += on[p] ? v : 0.0f;
            }
            if constexpr (!XW) part = wave_sum(part);
        }
        if constexpr (XW) {
            // the row's first wave adds the lane values of passes 0..3 in
            // order from 0, as the one-wave loop does, then the wave sum
            __syncthreads();
            if (seg == 0 && valid) {
                float t = 0.0f;
#pragma unroll
                for (int w = 0; w < WPR; ++w)
#pragma unroll
                    for (int p = 0; p < PASSES; ++p) t += xr[wid + w][p][lane];
                t = wave_sum(t);
                if (lane == 0) {
                    const float* bm = job.bias[m];
                    job.y[m][lr] = bm ? t + bm[lr] : t;
                }
            }
            __syncthreads();  // xr is rewritten by the next group
        } else if constexpr (!PAIR && WPR == 1) {
            if (valid && lane == 0) {
                const float* bm = job.bias[m];
                job.y[m][lr] = bm ? part + bm[lr] : part;
            }
        } else {
            if (lane == 0) red[wid] = part;
            __syncthreads();
            if constexpr (PAIR) {
                if (seg == 0 && rslot < kOutPerGroup && lane == 0 && valid) {
                    float gs = red[wid], us = red[wid + kOutPerGroup * WPR];
#pragma unroll
                    for (int s = 1; s < WPR; ++s) gs += red[wid + s], us += red[wid + kOutPerGroup * WPR + s];
                    const float act = silu_mul(gs, us);
                    job.act16[o] = f32_to_f16_bits(act);
                    if (job.act32) job.act32[o] = act;
                }
            } else {
                if (seg == 0 && lane == 0 && valid) {
                    float t = red[wid];
#pragma unroll
                    for (int s = 1; s < WPR; ++s) t += red[wid + s];
                    const float* bm = job.bias[m];
                    job.y[m][lr] = bm ? t + bm[lr] : t;
                }
            }
            __syncthreads();  // red[] is rewritten by the next group
        }
    };
    // The first group's chunks (NORM: loaded in the prologue) go out right
    // behind x's loads, unconditionally (row_of clamps), so the column
    // biases wait for x alone and the chunks stay in flight meanwhile.
    if constexpr (NORM == 0) {
        int64_t o, lr, a0;
        int m, nch;
        uint32_t delta;
        row_of(blockIdx.x, &o, &m, &lr);
        seg_of(lr, &a0, &nch, &delta);
        load_seg(job.W[m], a0, nch, ch);
        __builtin_amdgcn_sched_barrier(0);
        load_x_bias<PASSES>(xh, kb);
    }
    if constexpr (PF) {  // every later group's chunks a group ahead
        for (int64_t g = blockIdx.x; g * kOutPerGroup < n_out; g += gridDim.x) run_group(g, std::true_type{});
    } else {
        int64_t g = blockIdx.x;
        if (g * kOutPerGroup < n_out) run_group(g, std::true_type{});  // workgroup-uniform
        g += gridDim.x;
        for (; g * kOutPerGroup < n_out; g += gridDim.x) run_group(g, std::false_type{});
    }
    if constexpr (CLOCK)
        wave_clock_leave(static_cast<int64_t>(blockIdx.x) * NW + wid, lane, (n_out + kOutPerGroup - 1) / kOutPerGroup);
}

// Pair kernel with one wave per output row, for rows of at most 16 blocks
// (q6_wpr == 1: one segment per row).  Wave w of the grid computes output
// rows o = w, w + W, w + 2W, .. (W waves in the grid): gate row o, then up
// row o, each staged through an LDS buffer of the wave's own and summed
// exactly as the staged kernel's one-wave rows are (passes in order, masked
// block slots adding +0, then the wave sum), and act = silu(g) * u in lane 0
// -- the staged pair kernel's values, bit for bit.  Gate and up meet in
// registers, so after the NORM prologue no wave waits for another; the staged
// pair layout puts a row's gate and up on different waves that meet in LDS
// behind two barriers per row group.  PF: the next output row's chunks are
// loaded as soon as the current row's are in LDS and stay in flight while it
// is computed.  NORM / VW: the staged kernel's prologue (RmsIn), for NW waves.
// CLOCK: the instrumented copy (FENCE_WAVE_CLOCK builds), whose row-group
// count is the wave's rows.
// MERGE (rows whose last pass holds two blocks, nb % 4 == 2): that pass is
// one pass for both rows -- block slots 0, 1 take gate's two blocks, slots
// 2, 3 up's -- and up's two values move to slots 0, 1 (a half-wave swap),
// where the unmerged layout computes them: each lane adds exactly the values
// it adds there, in the same order, so the sums are the same bits, from five
// passes per output row instead of six.
template <int PASSES, int NW, int NORM, int VW, bool PF, bool MERGE, bool CLOCK = false>
__global__ __launch_bounds__(kWave * NW) __attribute__((amdgpu_waves_per_eu(FENCE_GEMV_Q6K_PAIRW_WPE))) void gemv_q6k_pairw_kernel(const Q6Job job, const uint16_t* __restrict__ x16,
                                                                  int nb, const RmsIn rin) {
    static_assert(!MERGE || PASSES >= 2, "a merged last pass follows full ones");
    constexpr int kSegBytes = 4 * PASSES * kBlockBytes + 32;  // + alignment slack
    constexpr int kBufBytes = (kSegBytes + 15) / 16 * 16;
    constexpr int kChunkSlots = (kSegBytes / 16 + kWave - 1) / kWave;
    constexpr uint32_t kPassBytes = 4 * kBlockBytes;
    constexpr int kStageBytes = NW * 2 * kBufBytes;
    constexpr int kNormXBytes = 2 * 1024 * PASSES;
    constexpr int kLdsBytes = NORM && kNormXBytes > kStageBytes ? kNormXBytes : kStageBytes;
    __shared__ __align__(16) uint8_t lds[kLdsBytes];
    __shared__ float nred[NORM ? 16 : 1];
    const int lane = threadIdx.x & (kWave - 1);
    const int wid = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
    uint8_t* bufg = lds + wid * (2 * kBufBytes);
    uint8_t* bufu = bufg + kBufBytes;
    const int bslot = lane >> 4, h = (lane >> 3) & 1, j = lane & 7;
    const int b0 = 0, b1 = nb;
    const int64_t row_bytes = static_cast<int64_t>(nb) * kBlockBytes;
    const int64_t n_out = job.end[0];
    const int64_t waves = static_cast<int64_t>(gridDim.x) * NW;
    const int64_t o0 = static_cast<int64_t>(blockIdx.x) * NW + wid;
    if constexpr (CLOCK) wave_clock_enter(o0, lane);

    uint32_t xh[PASSES][8];
    float kb[PASSES][4];
    // MERGE: x of the merged pass's block, 4 (PASSES - 1) + (bslot & 1), for
    // every slot (the last pass of xh masks slots 2, 3)
    uint32_t xm[1][8];
    float km[1][4];
    const int b0m = 4 * (PASSES - 1) + (bslot & 1) - bslot;
    if constexpr (!NORM) {
        load_x<PASSES>(xh, kb, x16, b0, b1, bslot, h, j);
        if constexpr (MERGE) load_x<1>(xm, km, x16, b0m, b1, bslot, h, j);
    }

    static_assert(NORM == 0 || (VW >= 1 && VW * NW <= 16 + NW - 1), "VW: 1 .. ceil(16 / NW) slots");
    constexpr int kVW = NORM ? VW : 1;
    constexpr int kVpt = NORM ? NORM : 1;
    f4 nh[kVW][kVpt], nr[kVW][kVpt], nw[kVW][kVpt];
    auto norm_slot = [&](int i, int jj, int* f) {
        const int vw = wid + NW * i;
        *f = vw * kWave + lane + jj * rin.T;
        return vw * kWave < rin.T && *f < nb * 64;
    };
    if constexpr (NORM != 0) {
        const float* rp = rin.res ? rin.res : rin.hid;
#pragma unroll
        for (int i = 0; i < kVW; ++i) {
#pragma unroll
            for (int jj = 0; jj < kVpt; ++jj) {
                int f;
                const int fc = norm_slot(i, jj, &f) ? f : 0;
                nh[i][jj] = ld4<false>(rin.hid + 4 * fc);
                nr[i][jj] = ld4<false>(rp + 4 * fc);
                nw[i][jj] = ld4<false>(rin.w + 4 * fc);
            }
        }
    }
    bool on[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; ++p) on[p] = b0 + 4 * p + bslot < b1;
    const uint32_t lane_ql = 64 * h + 4 * j;
    const uint32_t lane_qh = 128 + 32 * h + 4 * j;
    const uint32_t lane_sc = 192 + 8 * h + (j >> 2);
    const uint32_t blk_off = static_cast<uint32_t>(bslot) * kBlockBytes;

    // The 16-byte chunks covering row lr (the same for gate and up, which
    // share the shape): [a0, a0 + 16 * nch) of either matrix.
    auto seg_of = [&](int64_t lr, int64_t* a0, int* nch, uint32_t* delta) {
        const int64_t start = lr * row_bytes;
        const int64_t end = start + row_bytes;
        *a0 = start & ~int64_t(15);
        *nch = static_cast<int>((end - *a0 + 15) >> 4);
        *delta = static_cast<uint32_t>(start - *a0);
    };
    auto load_seg = [&](const uint8_t* Wm, int64_t a0, int nch, u4* ch) {
        const uint8_t* src = Wm + a0;
#pragma unroll
        for (int k = 0; k < kChunkSlots; ++k) {
            const int cc = lane + kWave * k;
            uint32_t off = 16u * static_cast<uint32_t>(cc < nch ? cc : 0);
            asm volatile("" : "+v"(off));
            ch[k] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(src + off));
        }
    };
    auto stage = [&](uint8_t* buf, int nch, const u4* ch) {
#pragma unroll
        for (int k = 0; k < kChunkSlots; ++k) {
            const int cc = lane + kWave * k;
            // a lane past the row's last chunk stores into the slack at the
            // buffer's end, which holds no block data
            const uint32_t dst = cc < nch ? 16u * cc : static_cast<uint32_t>(kBufBytes - 16);
            *reinterpret_cast<u4*>(buf + dst) = ch[k];
        }
    };
    // The lane's value of the block staged at byte `base` of buf (pass offset
    // included), against x pairs xp and biases kp.
    auto block_value = [&](const uint8_t* buf, uint32_t base, const uint32_t* xp, const float* kp) {
        const uint32_t sh = base & 3u;
        const uint8_t* ab = buf + (base & ~3u);
        const uint8_t* bb = buf + base;
        const uint32_t* wa = reinterpret_cast<const uint32_t*>(ab + lane_ql);
        const uint32_t* wb = reinterpret_cast<const uint32_t*>(ab + lane_ql + 32);
        const uint32_t* wc = reinterpret_cast<const uint32_t*>(ab + lane_qh);
        const uint32_t a = __builtin_amdgcn_alignbyte(wa[1], wa[0], sh);
        const uint32_t bq = __builtin_amdgcn_alignbyte(wb[1], wb[0], sh);
        const uint32_t c = __builtin_amdgcn_alignbyte(wc[1], wc[0], sh);
        const int8_t* scb = reinterpret_cast<const int8_t*>(bb + lane_sc);
        int sc[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) sc[q] = scb[2 * q];
        const uint16_t dbits = *reinterpret_cast<const uint16_t*>(bb + 208);
        const _Float16 d = __builtin_bit_cast(_Float16, dbits);
        return q6_lane_dot(q6_unpack(a, bq, c), xp, kp, sc, d);
    };
    // The lane's sum over the first NP passes of the row staged in buf, in
    // the staged kernel's order.  MERGE's first PASSES - 1 passes hold four
    // blocks each: no slot is masked there.
    auto row_part = [&](const uint8_t* buf, uint32_t delta, auto np) {
        constexpr bool kFull = MERGE && decltype(np)::value < PASSES;
        float part = 0.0f;
#pragma unroll
        for (int p = 0; p < decltype(np)::value; ++p) {
            const float v = block_value(buf, delta + blk_off + p * kPassBytes, xh[p], kb[p]);
            part += kFull || on[p] ? v : 0.0f;
        }
        return part;
    };

    u4 chg[kChunkSlots], chu[kChunkSlots];
    auto load_row = [&](int64_t o) {
        int64_t a0;
        int nch;
        uint32_t delta;
        seg_of(o < n_out ? o : n_out - 1, &a0, &nch, &delta);
        load_seg(job.W[0], a0, nch, chg);
        load_seg(job.W[1], a0, nch, chu);
    };
    // The first row's chunks go out before anything else waits, whether or
    // not the wave has a row (load_row clamps to the last): with no branch
    // around them the prologue's waits count them exactly and leave them in
    // flight.
    load_row(o0);
    if constexpr (NORM != 0) {
        const int nvw = rin.T / kWave;
        const bool has_res = rin.res != nullptr;
#pragma unroll
        for (int i = 0; i < kVW; ++i) {
#pragma unroll
            for (int jj = 0; jj < kVpt; ++jj) {
                int f;
                const bool ok = norm_slot(i, jj, &f);
                const f4 hv = has_res ? nh[i][jj] + nr[i][jj] : nh[i][jj];
                nh[i][jj] = ok ? hv : f4(0.0f);
                if (blockIdx.x == 0 && has_res && ok) st4<false>(rin.hid_out + 4 * f, hv);
            }
        }
#pragma unroll
        for (int i = 0; i < kVW; ++i) {
            const int vw = wid + NW * i;
            if (vw < nvw) {
                float ss = 0.0f;
                ss += dot4(nh[i][0]);
                ss += kVpt > 1 ? dot4(nh[i][kVpt - 1]) : 0.0f;
                ss = wave_reduce(ss, OpAdd{});
                if (lane == 0) nred[vw] = ss;
            }
        }
#pragma unroll
        for (int i = 0; i < kVW; ++i)
#pragma unroll
            for (int jj = 0; jj < kVpt; ++jj) nw[i][jj] = nw[i][jj] * nh[i][jj];
        __syncthreads();
        float tot = nred[0];
        for (int v = 1; v < nvw; ++v) tot += nred[v];
        const float rs = rsqrtf(tot / static_cast<float>(nb * 256) + rin.eps);
        uint16_t* xs = reinterpret_cast<uint16_t*>(lds);
#pragma unroll
        for (int i = 0; i < kVW; ++i) {
#pragma unroll
            for (int jj = 0; jj < kVpt; ++jj) {
                int f;
                if (norm_slot(i, jj, &f)) {
                    const f4 o = nw[i][jj] * rs;  // (w * h) * rs
                    st_h4<false>(xs + 4 * f, o);
                    if (blockIdx.x == 0) st_h4<false>(rin.x_out + 4 * f, o);
                }
            }
        }
        __syncthreads();
        load_x<PASSES>(xh, kb, xs, b0, b1, bslot, h, j);
        if constexpr (MERGE) load_x<1>(xm, km, xs, b0m, b1, bslot, h, j);
        __syncthreads();  // lds holds staged rows from here on
    }
    for (int64_t o = o0; o < n_out; o += waves) {  // wave-uniform
        int64_t a0;
        int nch;
        uint32_t delta;
        seg_of(o, &a0, &nch, &delta);
        if (!PF && o != o0) load_row(o);
        __builtin_amdgcn_sched_barrier(0);
        stage(bufg, nch, chg);
        stage(bufu, nch, chu);
        if constexpr (PF) {
            if (o + waves < n_out) {
                load_row(o + waves);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        float gs, us;
        if constexpr (MERGE) {
            using Full = std::integral_constant<int, PASSES - 1>;
            const float gp = row_part(bufg, delta, Full{});
            const float up = row_part(bufu, delta, Full{});
            // the merged pass: slots 0, 1 gate's blocks, slots 2, 3 up's
            const float vm = block_value(bslot < 2 ? bufg : bufu,
                                         delta + (bslot & 1) * kBlockBytes + (PASSES - 1) * kPassBytes, xm[0], km[0]);
            // up's values to slots 0, 1: y's lower half takes x's upper half
            float x = vm, y = vm;
            asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(x), "+v"(y));
            gs = wave_sum(gp + (bslot < 2 ? vm : 0.0f));
            us = wave_sum(up + (bslot < 2 ? y : 0.0f));
        } else {
            using All = std::integral_constant<int, PASSES>;
            gs = wave_sum(row_part(bufg, delta, All{}));
            us = wave_sum(row_part(bufu, delta, All{}));
        }
        if (lane == 0) {
            const float act = silu_mul(gs, us);
            job.act16[o] = f32_to_f16_bits(act);
            if (job.act32) job.act32[o] = act;
        }
    }
    if constexpr (CLOCK) wave_clock_leave_n(o0, lane, o0 < n_out ? (n_out - o0 + waves - 1) / waves : 0);
}

// The lane's value of block b of row lr (its 16 weights), for the direct
// kernel: dwords straight from global memory, two aligned dwords each,
// realigned.
__device__ __forceinline__ float direct_block(const uint8_t* Wm, const uint16_t* x16, int64_t lr, int nb, int b,
                                              int h, int j) {
    const uint8_t* blk = Wm + lr * static_cast<int64_t>(nb) * kBlockBytes + static_cast<int64_t>(b) * kBlockBytes;
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
    const _Float16 d = __builtin_bit_cast(_Float16, dbits);
    return q6_lane_dot(q6_unpack(a, bq, c), xh, kbc, sc, d);
}

// y . row lr of Wm (lane 0 holds it), summed in the order of q6_wpr /
// q6_passes -- the staged kernel's -- one segment after another.
__device__ __forceinline__ float direct_row(const uint8_t* Wm, const uint16_t* x16, int64_t lr, int nb, int lane) {
    const int bslot = lane >> 4, h = (lane >> 3) & 1, j = lane & 7;
    const int wpr = q6_wpr(nb), passes = q6_passes(nb);
    float total = 0.0f;
    for (int seg = 0; seg < wpr; ++seg) {
        int b0, b1;
        segment(nb, seg, wpr, &b0, &b1);
        float part = 0.0f;
        for (int p = 0; p < passes; ++p) {
            const int b = b0 + 4 * p + bslot;
            part += b < b1 ? direct_block(Wm, x16, lr, nb, b, h, j) : 0.0f;  // a masked slot adds +0
        }
        part = wave_sum(part);
        total = seg == 0 ? part : total + part;
    }
    return total;
}

// Direct kernel for any alignment and any K: one wave per row (PAIR: per
// output row, its gate row then its up row).
template <bool PAIR>
__global__ __launch_bounds__(kThreads) void gemv_q6k_direct_kernel(const Q6Job job,
                                                                   const uint16_t* __restrict__ x16, int nb) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t wave = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) / kWave;
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * (kThreads / kWave);
    const int64_t n_out = PAIR ? job.end[0] : job.end[job.n - 1];
    for (int64_t r = wave; r < n_out; r += nwaves) {
        if constexpr (PAIR) {
            const float gs = direct_row(job.W[0], x16, r, nb, lane);
            const float us = direct_row(job.W[1], x16, r, nb, lane);
            if (lane == 0) {
                const float act = silu_mul(gs, us);
                job.act16[r] = f32_to_f16_bits(act);
                if (job.act32) job.act32[r] = act;
            }
        } else {
            int64_t lr;
            const int m = mat_of(job, r, &lr);
            const float part = direct_row(job.W[m], x16, lr, nb, lane);
            if (lane == 0) {
                const float* bm = job.bias[m];
                job.y[m][lr] = bm ? part + bm[lr] : part;
            }
        }
    }
}

// A resident grid of `threads`-lane workgroups for `occ_kernel`: CUs x its
// occupancy per CU (cached per device in `cache`), at most `groups`; launches
// `kernel` on it (the same kernel, or its instrumented copy).
template <class OccKernel, class Kernel, class... Args>
int launch_grid_as(OccKernel occ_kernel, Kernel kernel, int threads, std::atomic<int>* cache, int64_t groups,
                   hipStream_t s, const Args&... args) {
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_status(e);
    if (dev < 0 || dev >= 64) return FENCE_ERROR_INVALID_VALUE;
    int g = cache[dev].load(std::memory_order_relaxed);
    if (g == 0) {
        int cus = 0, per_cu = 0;
        if (hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev); e != hipSuccess)
            return hip_status(e);
        if (hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, occ_kernel, threads, 0);
            e != hipSuccess)
            return hip_status(e);
        if (FENCE_GEMV_Q6K_WG_PER_CU > 0 && per_cu > FENCE_GEMV_Q6K_WG_PER_CU) per_cu = FENCE_GEMV_Q6K_WG_PER_CU;
        g = cus * (per_cu > 0 ? per_cu : 1);
        cache[dev].store(g, std::memory_order_relaxed);
    }
    if (!FENCE_GEMV_Q6K_RESIDENT) g = 0x7fffffff;
    int64_t w = groups < g ? groups : g;
    if (FENCE_GEMV_Q6K_BALANCED && w > 0) {
        const int64_t rounds = (groups + w - 1) / w;
        w = (groups + rounds - 1) / rounds;
    }
    const unsigned grid = static_cast<unsigned>(w);
    return launch(kernel, dim3(grid), dim3(threads), 0, s, args...);
}

template <class Kernel, class... Args>
int launch_grid(Kernel kernel, int threads, std::atomic<int>* cache, int64_t groups, hipStream_t s,
                const Args&... args) {
    return launch_grid_as(kernel, kernel, threads, cache, groups, s, args...);
}

template <int PASSES, int WPR, bool PAIR, bool MULTI, int NORM, bool XW, int VW>
int launch_staged_vw(const Q6Job& job, int64_t n_out, const uint16_t* x, int nb, const RmsIn& rin, hipStream_t s) {
    static std::atomic<int> cache[64];
    constexpr int nw = staged_waves<WPR, PAIR, NORM>();
    constexpr int out_per_group = PAIR ? nw / WPR / 2 : nw / WPR;
    return launch_grid_as(gemv_q6k_staged_kernel<PASSES, WPR, PAIR, MULTI, NORM, XW, false, VW>,
                          gemv_q6k_staged_kernel<PASSES, WPR, PAIR, MULTI, NORM, XW, FENCE_WAVE_CLOCK != 0, VW>,
                          kWave * nw, cache, (n_out + out_per_group - 1) / out_per_group, s, job, x, nb, rin);
}

template <int PASSES, int WPR, bool PAIR, bool MULTI, int NORM, bool XW = false>
int launch_staged(const Q6Job& job, int64_t n_out, const uint16_t* x, int nb, const RmsIn& rin, hipStream_t s) {
    if constexpr (NORM == 0) {
        return launch_staged_vw<PASSES, WPR, PAIR, MULTI, NORM, XW, 0>(job, n_out, x, nb, rin, s);
    } else {
        constexpr int nw = staged_waves<WPR, PAIR, NORM>();
        const int vw = (rin.T / kWave + nw - 1) / nw;  // rin.T <= 1024: at most 16 / nw
        if (vw <= 1) return launch_staged_vw<PASSES, WPR, PAIR, MULTI, NORM, XW, 1>(job, n_out, x, nb, rin, s);
        if (vw == 2 || nw == 8) return launch_staged_vw<PASSES, WPR, PAIR, MULTI, NORM, XW, 2>(job, n_out, x, nb, rin, s);
        if constexpr (nw == 4) {
            if (vw == 3) return launch_staged_vw<PASSES, WPR, PAIR, MULTI, NORM, XW, 3>(job, n_out, x, nb, rin, s);
            return launch_staged_vw<PASSES, WPR, PAIR, MULTI, NORM, XW, 4>(job, n_out, x, nb, rin, s);
        }
        return FENCE_ERROR_INVALID_VALUE;  // not reached: nw is 4 or 8
    }
}

// The one-wave pair kernel (FENCE_GEMV_Q6K_PAIRW waves per workgroup) for
// rows of nb <= 16 blocks, on a resident grid.
template <int PASSES, int NORM, int VW>
int launch_pairw_vw(const Q6Job& job, int64_t n_out, const uint16_t* x, int nb, const RmsIn& rin, hipStream_t s) {
    constexpr int nw = FENCE_GEMV_Q6K_PAIRW > 0 ? FENCE_GEMV_Q6K_PAIRW : 4;
    static std::atomic<int> cache[64];
    constexpr bool pf = FENCE_GEMV_Q6K_PAIRW_PF != 0;
    if constexpr (PASSES >= 2 && FENCE_GEMV_Q6K_PAIRW_MERGE) {
        if (nb % 4 == 2) {
            static std::atomic<int> mcache[64];
            return launch_grid_as(gemv_q6k_pairw_kernel<PASSES, nw, NORM, VW, pf, true, false>,
                                  gemv_q6k_pairw_kernel<PASSES, nw, NORM, VW, pf, true, FENCE_WAVE_CLOCK != 0>,
                                  kWave * nw, mcache, (n_out + nw - 1) / nw, s, job, x, nb, rin);
        }
    }
    return launch_grid_as(gemv_q6k_pairw_kernel<PASSES, nw, NORM, VW, pf, false, false>,
                          gemv_q6k_pairw_kernel<PASSES, nw, NORM, VW, pf, false, FENCE_WAVE_CLOCK != 0>, kWave * nw, cache,
                          (n_out + nw - 1) / nw, s, job, x, nb, rin);
}

template <int PASSES, int NORM>
int launch_pairw_p(const Q6Job& job, int64_t n_out, const uint16_t* x, int nb, const RmsIn& rin, hipStream_t s) {
    if constexpr (NORM == 0) {
        return launch_pairw_vw<PASSES, 0, 0>(job, n_out, x, nb, rin, s);
    } else {
        constexpr int nw = FENCE_GEMV_Q6K_PAIRW > 0 ? FENCE_GEMV_Q6K_PAIRW : 4;
        const int vw = (rin.T / kWave + nw - 1) / nw;  // rin.T <= 1024: at most 16 / nw
        if (vw <= 1) return launch_pairw_vw<PASSES, NORM, 1>(job, n_out, x, nb, rin, s);
        if (vw == 2) return launch_pairw_vw<PASSES, NORM, 2>(job, n_out, x, nb, rin, s);
        if constexpr (3 * nw <= 16 + nw - 1) {
            if (vw == 3) return launch_pairw_vw<PASSES, NORM, 3>(job, n_out, x, nb, rin, s);
        }
        if constexpr (4 * nw <= 16 + nw - 1) {
            if (vw == 4) return launch_pairw_vw<PASSES, NORM, 4>(job, n_out, x, nb, rin, s);
        }
        return FENCE_ERROR_INVALID_VALUE;  // not reached: vw <= ceil(16 / nw)
    }
}

template <int NORM>
int launch_pairw(const Q6Job& job, int64_t n_out, const uint16_t* x, int nb, const RmsIn& rin, hipStream_t s) {
    switch (q6_passes(nb)) {  // nb <= 16: one segment of 1-4 passes
        case 1: return launch_pairw_p<1, NORM>(job, n_out, x, nb, rin, s);
        case 2: return launch_pairw_p<2, NORM>(job, n_out, x, nb, rin, s);
        case 3: return launch_pairw_p<3, NORM>(job, n_out, x, nb, rin, s);
        case 4: return launch_pairw_p<4, NORM>(job, n_out, x, nb, rin, s);
        default: return FENCE_ERROR_INVALID_VALUE;  // not reached for nb <= 16
    }
}

// Whether a pair of rows of nb blocks takes the one-wave pair kernel.
constexpr bool use_pairw(int nb) { return FENCE_GEMV_Q6K_PAIRW != 0 && nb <= 16 && q6_wpr(nb) == 1; }

// The staged kernel for a row of nb blocks, at q6_wpr / q6_passes.  Only the
// (PASSES, WPR) pairs the compiled split table produces are instantiated; NORM
// launches take rows of up to 32 blocks.
template <bool PAIR, bool MULTI, int NORM>
int launch_nb(const Q6Job& job, int64_t n_out, const uint16_t* x, int nb, const RmsIn& rin, hipStream_t s) {
    const int w = q6_wpr(nb), p = q6_passes(nb);
    if (nb > 4 * kMaxSegBlocks || (NORM != 0 && nb > 32)) return FENCE_ERROR_INVALID_VALUE;  // callers check nb
#define FENCE_Q6_STAGED(P, W)                                                   \
    if (p == P && w == W) return launch_staged<P, W, PAIR, MULTI, NORM>(job, n_out, x, nb, rin, s);
    if constexpr (FENCE_GEMV_Q6K_SPLIT == 2) {
        FENCE_Q6_STAGED(1, 1) FENCE_Q6_STAGED(1, 2) FENCE_Q6_STAGED(1, 4) FENCE_Q6_STAGED(2, 4)
    } else if constexpr (FENCE_GEMV_Q6K_SPLIT == 1) {
        FENCE_Q6_STAGED(1, 1) FENCE_Q6_STAGED(2, 1) FENCE_Q6_STAGED(2, 2) FENCE_Q6_STAGED(2, 4)
    } else {
        FENCE_Q6_STAGED(1, 1) FENCE_Q6_STAGED(2, 1) FENCE_Q6_STAGED(3, 1) FENCE_Q6_STAGED(4, 1)
        FENCE_Q6_STAGED(3, 2) FENCE_Q6_STAGED(4, 2)
    }
    if constexpr (NORM == 0) {
        FENCE_Q6_STAGED(3, 4) FENCE_Q6_STAGED(4, 4)
        if constexpr (FENCE_GEMV_Q6K_SPLIT == 0 && FENCE_GEMV_Q6K_WIDE) {
            FENCE_Q6_STAGED(5, 2)
        }
    }
#undef FENCE_Q6_STAGED
    return FENCE_ERROR_INVALID_VALUE;  // a pair the table cannot produce
}

template <bool PAIR>
int launch_direct(const Q6Job& job, int64_t n_out, const uint16_t* x, int nb, hipStream_t s) {
    static std::atomic<int> cache[64];
    return launch_grid(gemv_q6k_direct_kernel<PAIR>, kThreads, cache, (n_out + 3) / 4, s, job, x, nb);
}

// Checks and dispatch of a job whose matrices, rows and outputs are filled in.
// With `rin` (checked by rms_input) x is computed from it: in the GEMV's own
// prologue where the row norm would run its vector kernel at a shape the
// prologue takes, otherwise by that kernel into rin->x_out first.
int gemv_q6k_run(Q6Job& job, const void* xv, int K, bool pair, hipStream_t s, const RmsIn* rin = nullptr) {
    if (K <= 0 || (K % 256) != 0) return FENCE_ERROR_INVALID_VALUE;
    if (!rin && (!xv || !aligned(xv, 2))) return FENCE_ERROR_INVALID_VALUE;
    const int nb = K / 256;
    const int64_t n_out = pair ? job.end[0] : job.end[job.n - 1];
    if (n_out == 0)  // no rows: the input row is still produced
        return rin ? residual_rms_f16_launch(rin->hid_out, rin->x_out, rin->hid, rin->res, rin->w, K, rin->eps, s)
                   : FENCE_SUCCESS;
    bool staged = nb <= 4 * kMaxSegBlocks;
    int prev = 0;
    for (int i = 0; i < job.n; ++i) {
        const int rows = job.end[i] - prev;
        prev = job.end[i];
        if (rows == 0) continue;
        staged = staged && aligned(job.W[i], 16) && (static_cast<int64_t>(rows) * nb) % 8 == 0;
    }
    const RmsIn none{};
    if (rin) {
        RmsIn r = *rin;
        unsigned T = 0;
        const bool vec_norm = aligned(r.hid, 16) && aligned(r.w, 16) && aligned(r.x_out, 8) &&
                              (!r.res || (aligned(r.res, 16) && aligned(r.hid_out, 16)));
        // Two float4 per lane double the prologue's registers: measured on
        // MI355X, q/k/v at K = 5120 still gain (18.8 -> 15.2 us against the
        // two launches) but gate/up, whose workgroups loop over many more row
        // groups, lose at the lower occupancy (40.8 -> 48.2 us), so a pair
        // takes the two launches there.
        if (staged && nb <= 32 && vec_norm && rms_row_plan(1, K, &T, &r.vpt) && T <= 1024 &&
            (r.vpt == 1 || (r.vpt == 2 && !pair))) {
            r.T = static_cast<int>(T);
            if (r.vpt == 1) {
                if (pair && use_pairw(nb)) return launch_pairw<1>(job, n_out, nullptr, nb, r, s);
                return pair ? launch_nb<true, false, 1>(job, n_out, nullptr, nb, r, s)
                            : launch_nb<false, true, 1>(job, n_out, nullptr, nb, r, s);
            }
            return launch_nb<false, true, 2>(job, n_out, nullptr, nb, r, s);
        }
        if (int st = residual_rms_f16_launch(r.hid_out, r.x_out, r.hid, r.res, r.w, K, r.eps, s)) return st;
        xv = r.x_out;
    }
    const uint16_t* x = static_cast<const uint16_t*>(xv);
    if (pair) {
        if (staged && use_pairw(nb)) return launch_pairw<0>(job, n_out, x, nb, none, s);
        return staged ? launch_nb<true, false, 0>(job, n_out, x, nb, none, s) : launch_direct<true>(job, n_out, x, nb, s);
    }
    if (!staged) return launch_direct<false>(job, n_out, x, nb, s);
    // Few rows of 13-16 blocks: one wave per row leaves most SIMDs idle, so
    // the one-wave layout runs spread over four waves per row (bit-identical).
    if (FENCE_GEMV_Q6K_SPLIT == 0 && nb > 12 && nb <= 16 && n_out <= FENCE_GEMV_Q6K_XW_ROWS)
        return job.n > 1 ? launch_staged<1, 4, false, true, 0, true>(job, n_out, x, nb, none, s)
                         : launch_staged<1, 4, false, false, 0, true>(job, n_out, x, nb, none, s);
    return job.n > 1 ? launch_nb<false, true, 0>(job, n_out, x, nb, none, s)
                     : launch_nb<false, false, 0>(job, n_out, x, nb, none, s);
}

// Whether byte ranges [a, a + an) and [b, b + bn) share a byte (null: no).
bool overlap(const void* a, size_t an, const void* b, size_t bn) {
    if (!a || !b) return false;
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + bn && y < x + an;
}

// A fence_rms_input for rows of K floats: required pointers, alignment, and
// no output overlapping an input (workgroup 0 writes them while the others
// read).
int rms_input(const fence_rms_input* in, int K, RmsIn* r) {
    if (!in || !in->hidden || !in->weight || !in->x_f16 || (in->residual && !in->hidden_out))
        return FENCE_ERROR_INVALID_VALUE;
    if (!aligned(in->hidden, 4) || !aligned(in->weight, 4) || !aligned(in->x_f16, 2) ||
        (in->residual && (!aligned(in->residual, 4) || !aligned(in->hidden_out, 4))))
        return FENCE_ERROR_INVALID_VALUE;
    const size_t f = static_cast<size_t>(K) * 4, hb = static_cast<size_t>(K) * 2;
    float* hout = in->residual ? in->hidden_out : nullptr;
    if (overlap(hout, f, in->hidden, f) || overlap(hout, f, in->residual, f) || overlap(hout, f, in->weight, f) ||
        overlap(in->x_f16, hb, in->hidden, f) || overlap(in->x_f16, hb, in->residual, f) ||
        overlap(in->x_f16, hb, in->weight, f) || overlap(in->x_f16, hb, hout, f))
        return FENCE_ERROR_INVALID_VALUE;
    *r = RmsIn{in->hidden, in->residual, hout, in->weight, static_cast<uint16_t*>(in->x_f16), in->eps, 0, 0};
    return FENCE_SUCCESS;
}

int gemv_q6k_launch(float* y, const void* Wv, const void* xv, const float* bias, int M, int K, hipStream_t s) {
    if (M < 0 || K < 0 || (K % 256) != 0) return FENCE_ERROR_INVALID_VALUE;
    if (M == 0) return FENCE_SUCCESS;
    if (K == 0 || !y || !Wv || !xv) return FENCE_ERROR_INVALID_VALUE;
    if (!aligned(Wv, 2) || !aligned(y, 4) || (bias && !aligned(bias, 4))) return FENCE_ERROR_INVALID_VALUE;
    Q6Job job{};
    job.W[0] = static_cast<const uint8_t*>(Wv);
    job.y[0] = y;
    job.bias[0] = bias;
    job.end[0] = M;
    job.n = 1;
    return gemv_q6k_run(job, xv, K, false, s);
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

namespace fence {
namespace {

// The job of a multi launch: n matrices of M[i] rows.
int multi_job(int n, const void* const* W, float* const* y, const float* const* bias, const int* M, Q6Job* job) {
    if (n < 1 || n > kMaxMats || !W || !y || !M) return FENCE_ERROR_INVALID_VALUE;
    *job = Q6Job{};
    int64_t total = 0;
    for (int i = 0; i < n; ++i) {
        if (M[i] < 0) return FENCE_ERROR_INVALID_VALUE;
        if (M[i] > 0 && (!W[i] || !y[i] || !aligned(W[i], 2) || !aligned(y[i], 4) ||
                         (bias && bias[i] && !aligned(bias[i], 4))))
            return FENCE_ERROR_INVALID_VALUE;
        total += M[i];
        if (total > 0x7fffffff) return FENCE_ERROR_INVALID_VALUE;
        job->W[i] = static_cast<const uint8_t*>(W[i]);
        job->y[i] = y[i];
        job->bias[i] = bias ? bias[i] : nullptr;
        job->end[i] = static_cast<int>(total);
    }
    job->n = n;
    return FENCE_SUCCESS;
}

// The job of a gate/up pair of M rows each.
int pair_job(const void* W_gate, const void* W_up, void* out_f16, float* out, int M, Q6Job* job) {
    if (M < 0 || M > 0x3fffffff) return FENCE_ERROR_INVALID_VALUE;
    if (M > 0 && (!W_gate || !W_up || !out_f16 || !aligned(W_gate, 2) || !aligned(W_up, 2) ||
                  !aligned(out_f16, 2) || (out && !aligned(out, 4))))
        return FENCE_ERROR_INVALID_VALUE;
    *job = Q6Job{};
    job->W[0] = static_cast<const uint8_t*>(W_gate);
    job->W[1] = static_cast<const uint8_t*>(W_up);
    job->end[0] = M;
    job->end[1] = 2 * M;  // rows of up follow gate's (row counts for the staging checks)
    job->n = 2;
    job->act16 = static_cast<uint16_t*>(out_f16);
    job->act32 = out;
    return FENCE_SUCCESS;
}

}  // namespace
}  // namespace fence

extern "C" int fence_gemv_q6k_multi(int n, const void* const* W, float* const* y, const float* const* bias,
                                    const int* M, const void* x, int K, hipStream_t stream) {
    using namespace fence;
    Q6Job job;
    if (int st = multi_job(n, W, y, bias, M, &job)) return st;
    if (K < 0 || K % 256 != 0) return FENCE_ERROR_INVALID_VALUE;
    if (job.end[n - 1] == 0) return FENCE_SUCCESS;
    return gemv_q6k_run(job, x, K, false, stream);
}

extern "C" int fence_gemv_q6k_swiglu_f16(const void* W_gate, const void* W_up, const void* x, void* out_f16,
                                         float* out, int M, int K, hipStream_t stream) {
    using namespace fence;
    Q6Job job;
    if (int st = pair_job(W_gate, W_up, out_f16, out, M, &job)) return st;
    if (K < 0 || K % 256 != 0) return FENCE_ERROR_INVALID_VALUE;
    if (M == 0) return FENCE_SUCCESS;
    return gemv_q6k_run(job, x, K, true, stream);
}

extern "C" int fence_gemv_q6k_multi_rms(int n, const void* const* W, float* const* y, const float* const* bias,
                                        const int* M, const fence_rms_input* in, int K, hipStream_t stream) {
    using namespace fence;
    Q6Job job;
    RmsIn r;
    if (int st = multi_job(n, W, y, bias, M, &job)) return st;
    if (K <= 0 || K % 256 != 0) return FENCE_ERROR_INVALID_VALUE;
    if (int st = rms_input(in, K, &r)) return st;
    return gemv_q6k_run(job, nullptr, K, false, stream, &r);
}

extern "C" int fence_gemv_q6k_swiglu_rms_f16(const void* W_gate, const void* W_up, const fence_rms_input* in,
                                             void* out_f16, float* out, int M, int K, hipStream_t stream) {
    using namespace fence;
    Q6Job job;
    RmsIn r;
    if (int st = pair_job(W_gate, W_up, out_f16, out, M, &job)) return st;
    if (K <= 0 || K % 256 != 0) return FENCE_ERROR_INVALID_VALUE;
    if (int st = rms_input(in, K, &r)) return st;
    return gemv_q6k_run(job, nullptr, K, true, stream, &r);
}

#if FENCE_WAVE_CLOCK
// Instrumented library only (include/fence/wave_clock.h).
extern "C" int fence_wave_clock_clear(void) {
    void* p = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(fence::wave_clock)); e != hipSuccess)
        return fence::hip_status(e);
    if (hipError_t e = hipMemset(p, 0, sizeof(fence::wave_clock)); e != hipSuccess) return fence::hip_status(e);
    return fence::hip_status(hipDeviceSynchronize());
}

extern "C" int fence_wave_clock_read(uint64_t* dst, int64_t max_waves) {
    if (!dst || max_waves < 0) return FENCE_ERROR_INVALID_VALUE;
    const int64_t n = max_waves < fence::kWaveClockMax ? max_waves : fence::kWaveClockMax;
    if (hipError_t e = hipDeviceSynchronize(); e != hipSuccess) return fence::hip_status(e);
    return fence::hip_status(hipMemcpyFromSymbol(dst, HIP_SYMBOL(fence::wave_clock), 32 * n, 0,
                                                 hipMemcpyDeviceToHost));
}
#endif
