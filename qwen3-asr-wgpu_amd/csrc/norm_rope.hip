// norm_rope.hip -- stage (a): fused q/k RMSNorm + rotate-half MRoPE + f16 KV
// append, one workgroup per row.
//
// Replaces the reference's qkv_extract / qkv_extract_slots WGSL kernels
// (src/shaders.rs:1376-1635) with the numerics of the CPU decoder
// (src/cpu_decoder.rs:274-290 norm_rope_head, 398-423 cache write), which it
// matches bit for bit: see norm_rope.hpp.
//
// Per row: the (nqh + nkvh) normed heads are staged in LDS with a padded
// stride (136 halves) so the per-head serial sum-of-squares lanes do not all
// hit one bank; gains and the row's cos/sin are staged too.  The work is
// HBM-bound and tiny (8 KiB in, 8 KiB out per row).

#include "kernels.hpp"
#include "norm_rope.hpp"

namespace qasr {

namespace {

constexpr int kRowThreads = 128;
constexpr int kMaxNormHeads = 48;  // nqh + nkvh
constexpr int kPad = kHeadDim + 8;

__global__ __launch_bounds__(kRowThreads) void norm_rope_append_kernel(
    CacheGeom g, int layer, SegPlan P, const f16* __restrict__ qkv,
    const f16* __restrict__ q_gain, const f16* __restrict__ k_gain,
    const f16* __restrict__ cos_tab, const f16* __restrict__ sin_tab, f16* __restrict__ q_out) {
    __shared__ __attribute__((aligned(16))) f16 s_raw[kMaxNormHeads * kPad];
    __shared__ __attribute__((aligned(16))) f16 s_aux[4 * kHeadDim];  // qg, kg, cos, sin
    __shared__ float s_inv[kMaxNormHeads];

    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    int sg = 0;
    while (sg + 1 < P.nseg && P.row_base[sg + 1] <= row) ++sg;
    const int pos = P.pos0[sg] + (row - P.row_base[sg]);
    const int slot = P.slot[sg];
    const int nqh = P.nqh, nkvh = g.nkvh;
    const int nh = nqh + nkvh;
    const int64_t tot = (int64_t)(nqh + 2 * nkvh) * kHeadDim;
    const f16* src = qkv + (int64_t)row * tot;

    for (int i = tid; i < nh * 16; i += kRowThreads) {
        const int h = i >> 4, w = (i & 15) * 8;
        *(uint4*)&s_raw[h * kPad + w] = *(const uint4*)(src + h * kHeadDim + w);
    }
    if (tid < 64) {
        const int which = tid >> 4, w = (tid & 15) * 8;
        const f16* p = which == 0 ? q_gain
                     : which == 1 ? k_gain
                     : which == 2 ? cos_tab + (int64_t)pos * kHeadDim
                                  : sin_tab + (int64_t)pos * kHeadDim;
        *(uint4*)&s_aux[which * kHeadDim + w] = *(const uint4*)(p + w);
    }
    __syncthreads();
    if (tid < nh) s_inv[tid] = head_inv_rms_serial(&s_raw[tid * kPad], P.eps);
    __syncthreads();

    const f16* crow = &s_aux[2 * kHeadDim];
    const f16* srow = &s_aux[3 * kHeadDim];
    f16* kdst = g.base + slot * g.slot_stride + layer * g.layer_stride + (int64_t)pos * kHeadDim;
    for (int it = tid; it < nh * 16; it += kRowThreads) {
        const int h = it >> 4, j0 = (it & 15) * 8;
        const bool is_q = h < nqh;
        const f16* gain = is_q ? &s_aux[0] : &s_aux[kHeadDim];
        const float inv = s_inv[h];
        H8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o.e[e] = rope_elem(&s_raw[h * kPad], gain, crow, srow, inv, j0 + e);
        if (is_q)
            *(uint4*)(q_out + (int64_t)row * nqh * kHeadDim + h * kHeadDim + j0) = o.u;
        else
            *(uint4*)(kdst + (h - nqh) * g.head_stride + j0) = o.u;
    }
    const f16* vsrc = src + (int64_t)(nqh + nkvh) * kHeadDim;
    f16* vdst = kdst + g.kv_stride;
    for (int it = tid; it < nkvh * 16; it += kRowThreads) {
        const int h = it >> 4, w = (it & 15) * 8;
        *(uint4*)(vdst + h * g.head_stride + w) = *(const uint4*)(vsrc + h * kHeadDim + w);
    }
}

}  // namespace

hipError_t launch_norm_rope_append(const CacheGeom& g, int layer, const SegPlan& P,
                                   const f16* qkv, const f16* q_gain, const f16* k_gain,
                                   const f16* cos_tab, const f16* sin_tab, f16* q_out,
                                   hipStream_t stream) {
    const int rows = P.row_base[P.nseg];
    if (rows <= 0) return hipSuccess;
    if (P.nqh + g.nkvh > kMaxNormHeads) return hipErrorInvalidValue;
    hipLaunchKernelGGL(norm_rope_append_kernel, dim3(rows), dim3(kRowThreads), 0, stream, g, layer,
                       P, qkv, q_gain, k_gain, cos_tab, sin_tab, q_out);
    return hipGetLastError();
}

}  // namespace qasr
