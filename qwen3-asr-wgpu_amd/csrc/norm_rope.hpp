// norm_rope.hpp -- per-head q/k RMSNorm + rotate-half RoPE, bit-identical to
// the reference CPU decoder's norm_rope_head (src/cpu_decoder.rs:274-290).
//
// Every float operation is written in the reference's order with contraction
// off, so each product and sum rounds exactly once, as in Rust:
//   sum2 = sequential sum over j of x_j*x_j            (277-281)
//   inv  = 1 / sqrt(sum2 / hd + eps)                   (282, IEEE div + sqrt)
//   xj   = (x_j * inv) * g_j ; xp = (x_pj * inv) * g_pj (284, 286)
//   out  = f16(xj*c_j + sign*xp*s_j)                   (288, RNE)
// HIP's default -fhip-fp32-correctly-rounded-divide-sqrt makes '/' and sqrtf
// correctly rounded; v_cvt_f16_f32 rounds to nearest even.
#pragma once

#include "common.hpp"

namespace qasr {

// The one serial chain of the stage, over squares already in LDS (sq[j] =
// x_j*x_j in f32, exact for an f16 x_j): only the 128 dependent adds in
// ascending j round, in the reference's order.  All 32 four-square reads are
// issued before the adds (one LDS latency, not one per read).
__device__ __forceinline__ float head_inv_rms_squares_all(const float* sq, float eps) {
#pragma clang fp contract(off)
    float4 v[kHeadDim / 4];
#pragma unroll
    for (int i = 0; i < kHeadDim / 4; ++i) v[i] = *(const float4*)(sq + 4 * i);
    float sum2 = 0.0f;
#pragma unroll
    for (int i = 0; i < kHeadDim / 4; ++i) {
        sum2 += v[i].x;
        sum2 += v[i].y;
        sum2 += v[i].z;
        sum2 += v[i].w;
    }
    return 1.0f / sqrtf(sum2 / (float)kHeadDim + eps);
}

// One roped element j of a head whose raw values, gains and cos/sin rows are
// given (all f16).  `inv` is the head's inverse RMS.
__device__ __forceinline__ f16 rope_elem(const f16* raw, const f16* gain, const f16* cos_row,
                                         const f16* sin_row, float inv, int j) {
#pragma clang fp contract(off)
    constexpr int half = kHeadDim / 2;
    const int pj = j < half ? j + half : j - half;
    const float xj = (h2f(raw[j]) * inv) * h2f(gain[j]);
    const float xp = (h2f(raw[pj]) * inv) * h2f(gain[pj]);
    const float a = xj * h2f(cos_row[j]);
    const float b = xp * h2f(sin_row[j]);
    // sign * xp * s with sign = -1 for j < half: (-xp)*s == -(xp*s) exactly.
    return f2h(j < half ? a - b : a + b);
}

// Elements j0 .. j0+7 (j0 a multiple of 8) of the same, each operand read as
// one 16-byte vector (the rotation partners j0 +- half are 8 aligned too);
// per element the arithmetic of rope_elem.
__device__ __forceinline__ uint4 rope8(const f16* raw, const f16* gain, const f16* cos_row,
                                       const f16* sin_row, float inv, int j0) {
#pragma clang fp contract(off)
    constexpr int half = kHeadDim / 2;
    const bool lo = j0 < half;
    const int p0 = lo ? j0 + half : j0 - half;
    H8 x, xp, g, gp, c, sn, o;
    x.u = *(const uint4*)(raw + j0);
    xp.u = *(const uint4*)(raw + p0);
    g.u = *(const uint4*)(gain + j0);
    gp.u = *(const uint4*)(gain + p0);
    c.u = *(const uint4*)(cos_row + j0);
    sn.u = *(const uint4*)(sin_row + j0);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float xj = (h2f(x.e[e]) * inv) * h2f(g.e[e]);
        const float xq = (h2f(xp.e[e]) * inv) * h2f(gp.e[e]);
        const float a = xj * h2f(c.e[e]);
        const float b = xq * h2f(sn.e[e]);
        o.e[e] = f2h(lo ? a - b : a + b);
    }
    return o.u;
}

}  // namespace qasr
