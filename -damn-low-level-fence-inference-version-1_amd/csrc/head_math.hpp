// head_math.hpp -- the per-head arithmetic of QK-norm and RoPE on gfx950,
// shared by the head kernels (head_ops.hip) and the attention kernel that
// prepares its own q and k (attention.hip), so that both round identically.
//
// Reference math:
//   per-head norm  rms_norm_per_head, src/kernels/ops.cuh:66-103:
//                  x = (w * x) * rsqrt(sum(x^2) / hd + eps)
//   RoPE           apply_rope, src/kernels/ops.cuh:115-177 (NeoX pairs (p, p + hd/2));
//                  interleaved pairs (2p, 2p + 1) of the comment at ops.cuh:109-113:
//                  x0' = x0 cos a - x1 sin a,  x1' = x0 sin a + x1 cos a,
//                  a = (float)pos * freq[p],  freq[p] = 1.0f / powf(base, (float)(2p) / (float)hd).
//
// A "unit" is the 8 floats one lane holds of one head: elements [4i, 4i + 4)
// and [hd/2 + 4i, hd/2 + 4i + 4), i < hd/8 -- four whole NeoX pairs, or four
// whole interleaved pairs -- so no lane needs a partner's values, and a
// head's hd/8 units sit in consecutive lanes (one 16-lane DPP row at hd = 128).
// The sums and rotations here are written with contraction off: their
// rounding does not depend on the kernel they are inlined into.
#pragma once

#include "common.hpp"

namespace fence {

enum { kRopeNone = -1, kRopeNeox = FENCE_ROPE_NEOX, kRopeInter = FENCE_ROPE_INTERLEAVED };

constexpr int kMaxHalf = 128;  // head_dim <= 256 for RoPE

// freq[p] of every pair, computed on the host (the reference's expression)
// and passed by value in the kernel arguments.
struct InvFreq {
    float v[kMaxHalf];
};

// Host: freq[p] = 1.0f / powf(base, (float)(2p) / (float)hd) for p < hd/2
// (ops.cuh:133), into out (head_ops.hip).
void rope_inv_freq_host(float* out, int hd, float base);

// sin and cos of an angle given in radians as an exact float (the angle
// (float)pos * freq[p], bit-identical to the reference's).  The angle is
// divided by pi and reduced to [-1, 1] in double -- error ~1e-16 for angles
// up to 2^24 rad -- and sincospif finishes in single precision with no
// large-argument reduction path.
__device__ __forceinline__ void sincos_angle(float a, float* s, float* c) {
    double t = static_cast<double>(a) * 0.31830988618379067154;  // 1/pi
    t -= 2.0 * __builtin_rint(t * 0.5);
    sincospif(static_cast<float>(t), s, c);
}

// rsqrt(sum of squares / n + eps), the per-head norm's scale.
__device__ __forceinline__ float head_rscale(float tot, float n, float eps) {
#pragma clang fp contract(off)
    return rsqrtf(tot / n + eps);
}

// The per-head norm of a unit: the head's sum of squares over its G lanes
// (a DPP reduction), then (w * x) * r.
template <int G>
__device__ __forceinline__ void head_norm_unit(f4& a, f4& b, f4 wa, f4 wb, float eps) {
    const float tot = group_reduce<G>(dot4(a) + dot4(b), OpAdd{});
    const float r = head_rscale(tot, static_cast<float>(8 * G), eps);
    a = (wa * a) * r;
    b = (wb * b) * r;
}

// One rotation: (x0 c - x1 s, x0 s + x1 c), two products and a sum each.
__device__ __forceinline__ f2 rope_pair(float x0, float x1, float c, float s) {
#pragma clang fp contract(off)
    f2 y;
    y.x = x0 * c - x1 * s;
    y.y = x0 * s + x1 * c;
    return y;
}

// RoPE of unit i of a head; cs = cos[half] then sin[half] of the token's
// pair angles (half = 4G).
template <int ROPE, int G>
__device__ __forceinline__ void rope_unit(f4& va, f4& vb, const float* cs, int i) {
    constexpr int HALF = 4 * G;
    if constexpr (ROPE == kRopeNeox) {
        const f4 c = *reinterpret_cast<const f4*>(cs + 4 * i);
        const f4 sn = *reinterpret_cast<const f4*>(cs + HALF + 4 * i);
        const f4 x0 = va, x1 = vb;
        const f2 r0 = rope_pair(x0.x, x1.x, c.x, sn.x), r1 = rope_pair(x0.y, x1.y, c.y, sn.y);
        const f2 r2 = rope_pair(x0.z, x1.z, c.z, sn.z), r3 = rope_pair(x0.w, x1.w, c.w, sn.w);
        va = f4{r0.x, r1.x, r2.x, r3.x};
        vb = f4{r0.y, r1.y, r2.y, r3.y};
    } else if constexpr (ROPE == kRopeInter) {
        // a holds pairs 2i, 2i + 1; b holds pairs HALF/2 + 2i, HALF/2 + 2i + 1
        const f2 ca = *reinterpret_cast<const f2*>(cs + 2 * i);
        const f2 sa = *reinterpret_cast<const f2*>(cs + HALF + 2 * i);
        const f2 cb = *reinterpret_cast<const f2*>(cs + HALF / 2 + 2 * i);
        const f2 sb = *reinterpret_cast<const f2*>(cs + HALF + HALF / 2 + 2 * i);
        const f2 a0 = rope_pair(va.x, va.y, ca.x, sa.x), a1 = rope_pair(va.z, va.w, ca.y, sa.y);
        const f2 b0 = rope_pair(vb.x, vb.y, cb.x, sb.x), b1 = rope_pair(vb.z, vb.w, cb.y, sb.y);
        va = f4{a0.x, a0.y, a1.x, a1.y};
        vb = f4{b0.x, b0.y, b1.x, b1.y};
    }
}

}  // namespace fence
