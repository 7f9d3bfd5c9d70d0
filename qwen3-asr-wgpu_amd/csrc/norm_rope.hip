// norm_rope.hip -- stage (a): fused q/k RMSNorm + rotate-half MRoPE + f16 KV
// append, one workgroup per row.
//
// Replaces the reference's qkv_extract / qkv_extract_slots WGSL kernels
// (src/shaders.rs:1376-1635) with the numerics of the CPU decoder
// (src/cpu_decoder.rs:274-290 norm_rope_head, 398-423 cache write), which it
// matches bit for bit: see norm_rope.hpp.
//
// Per row: the (nqh + nkvh) normed heads are staged in LDS with padded
// strides, their squares too, so the per-head serial sum lanes do not share a
// bank; gains and the row's cos/sin are staged as well.  The work is tiny
// (8 KiB in, 8 KiB out per row) and latency-bound.

#include "kernels.hpp"
#include "norm_rope.hpp"

namespace qasr {

namespace {

constexpr int kRowThreads = 384;  // one q/k piece per thread for 16 + 8 heads
constexpr int kMaxNormHeads = 48;  // nqh + nkvh
constexpr int kPad = kHeadDim + 8;    // f16 raw heads: padded rows
constexpr int kSqPad = kHeadDim + 4;  // f32 squares: lanes reading head h at the same j sit 4 banks apart

// Per row, one memory round trip and one serial chain: the raw q/k heads go
// to LDS (with their exact f32 squares, computed in parallel), the V heads to
// registers and straight back out to the cache; then one lane per head runs
// the reference's 128 dependent adds over the squares (all reads issued
// ahead of the adds), and the heads are normed, roped and written.
template <int QK>  // q/k 16-byte pieces per thread: ceil((nqh + nkvh) * 16 / kRowThreads)
__global__ __launch_bounds__(kRowThreads) void norm_rope_append_kernel(
    CacheGeom g, int layer, SegPlan P, const f16* __restrict__ qkv,
    const f16* __restrict__ q_gain, const f16* __restrict__ k_gain,
    const f16* __restrict__ cos_tab, const f16* __restrict__ sin_tab, f16* __restrict__ q_out) {
    __shared__ __attribute__((aligned(16))) f16 s_raw[kMaxNormHeads * kPad];
    __shared__ __attribute__((aligned(16))) float s_sq[kMaxNormHeads * kSqPad];
    __shared__ __attribute__((aligned(16))) f16 s_aux[4 * kHeadDim];  // qg, kg, cos, sin
    __shared__ float s_inv[kMaxNormHeads];

    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const int nqh = P.nqh, nkvh = g.nkvh;
    const int nh = nqh + nkvh;
    const int64_t tot = (int64_t)(nqh + 2 * nkvh) * kHeadDim;
    const f16* src = qkv + (int64_t)row * tot;

    // The row's loads first (they need only the row), all unconditional from
    // clamped in-row indices so they are in flight together: the q/k pieces
    // and V (one piece per thread of the last nv threads, so that wave 0,
    // which runs the serial chains, has no store outstanding).
    const int nqk = nh * 16, nv = nkvh * 16;
    uint4 x[QK];
#pragma unroll
    for (int k = 0; k < QK; ++k) {
        const int it = min(tid + k * kRowThreads, nqk - 1);
        x[k] = *(const uint4*)(src + (it >> 4) * kHeadDim + (it & 15) * 8);
    }
    const f16* vsrc = src + (int64_t)nh * kHeadDim;
    uint4 v;
    const int vt = tid - (kRowThreads - nv);  // V piece of this thread if >= 0
    {
        const int it = max(vt, 0);
        v = *(const uint4*)(vsrc + (it >> 4) * kHeadDim + (it & 15) * 8);
    }
    // Then the row's segment (position, slot) and the gains and cos/sin row.
    int sg = 0;
    while (sg + 1 < P.nseg && P.row_base[sg + 1] <= row) ++sg;
    const int pos = P.pos0[sg] + (row - P.row_base[sg]);
    const int slot = P.slot[sg];
    f16* kdst = g.base + slot * g.slot_stride + layer * g.layer_stride + (int64_t)pos * kHeadDim;
    f16* vdst = kdst + g.kv_stride;
    uint4 a;
    {
        const int which = (tid >> 4) & 3, w = (tid & 15) * 8;
        const f16* p = which == 0 ? q_gain
                     : which == 1 ? k_gain
                     : which == 2 ? cos_tab + (int64_t)pos * kHeadDim
                                  : sin_tab + (int64_t)pos * kHeadDim;
        a = *(const uint4*)(p + w);
    }
    // Keep every load here, issued back to back (the compiler would sink the
    // V load into its guarded store, a round trip of its own).
    asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
#pragma unroll
    for (int k = 0; k < QK; ++k) {
        const int it = tid + k * kRowThreads;
        if (it < nqk) {
            const int h = it >> 4, w = (it & 15) * 8;
            H8 y;
            y.u = x[k];
            *(uint4*)&s_raw[h * kPad + w] = y.u;
            float4 lo, hi;  // f16 squares are exact in f32
            lo.x = h2f(y.e[0]) * h2f(y.e[0]);
            lo.y = h2f(y.e[1]) * h2f(y.e[1]);
            lo.z = h2f(y.e[2]) * h2f(y.e[2]);
            lo.w = h2f(y.e[3]) * h2f(y.e[3]);
            hi.x = h2f(y.e[4]) * h2f(y.e[4]);
            hi.y = h2f(y.e[5]) * h2f(y.e[5]);
            hi.z = h2f(y.e[6]) * h2f(y.e[6]);
            hi.w = h2f(y.e[7]) * h2f(y.e[7]);
            *(float4*)&s_sq[h * kSqPad + w] = lo;
            *(float4*)&s_sq[h * kSqPad + w + 4] = hi;
        }
    }
    if (tid < 64) *(uint4*)&s_aux[(tid >> 4) * kHeadDim + (tid & 15) * 8] = a;
    if (vt >= 0) *(uint4*)(vdst + (vt >> 4) * g.head_stride + (vt & 15) * 8) = v;
    __syncthreads();
    if (tid < nh) s_inv[tid] = head_inv_rms_squares_all(&s_sq[tid * kSqPad], P.eps);
    __syncthreads();

    const f16* crow = &s_aux[2 * kHeadDim];
    const f16* srow = &s_aux[3 * kHeadDim];
    for (int it = tid; it < nh * 16; it += kRowThreads) {
        const int h = it >> 4, j0 = (it & 15) * 8;
        const bool is_q = h < nqh;
        const f16* gain = is_q ? &s_aux[0] : &s_aux[kHeadDim];
        const float inv = s_inv[h];
        const uint4 o = rope8(&s_raw[h * kPad], gain, crow, srow, inv, j0);
        if (is_q)
            *(uint4*)(q_out + (int64_t)row * nqh * kHeadDim + h * kHeadDim + j0) = o;
        else
            *(uint4*)(kdst + (h - nqh) * g.head_stride + j0) = o;
    }
}

}  // namespace

hipError_t launch_norm_rope_append(const CacheGeom& g, int layer, const SegPlan& P,
                                   const f16* qkv, const f16* q_gain, const f16* k_gain,
                                   const f16* cos_tab, const f16* sin_tab, f16* q_out,
                                   hipStream_t stream) {
    const int rows = P.row_base[P.nseg];
    if (rows <= 0) return hipSuccess;
    if (P.nqh < 1 || g.nkvh < 1 || P.nqh + g.nkvh > kMaxNormHeads || g.nkvh * 16 > kRowThreads)
        return hipErrorInvalidValue;
    const int nqk = (P.nqh + g.nkvh) * 16;
    static_assert(kMaxNormHeads * 16 <= 2 * kRowThreads, "two q/k pieces per thread at most");
    if (nqk <= kRowThreads)
        hipLaunchKernelGGL(norm_rope_append_kernel<1>, dim3(rows), dim3(kRowThreads), 0, stream, g,
                           layer, P, qkv, q_gain, k_gain, cos_tab, sin_tab, q_out);
    else
        hipLaunchKernelGGL(norm_rope_append_kernel<2>, dim3(rows), dim3(kRowThreads), 0, stream, g,
                           layer, P, qkv, q_gain, k_gain, cos_tab, sin_tab, q_out);
    return hipGetLastError();
}

}  // namespace qasr
