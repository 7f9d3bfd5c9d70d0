// diag.hip -- diagnostics and calibrations: qasr_softmax_weights (the
// attention kernels' softmax-weight exponent, common.hpp softmax_w_scaled /
// softmax_w_raw, over caller arrays, so tests can hold it against the
// reference's libm expf: cpu_decoder.rs:292-365 forms e = expf(s*scale -
// max*scale)), qasr_stream_read (a bare HBM stream) and qasr_mfma_probe (the
// matrix core's rate, the shader clock under load, and how much of the
// softmax's VALU work the matrix core hides).

#include "abi_internal.hpp"

using qasr::f16;
using qasr_abi::DeviceScope;
using qasr_abi::fail;
using qasr_abi::hip_fail;

namespace {

constexpr float kNegInfProbe = -__builtin_inff();

// out_scaled[i]: the decode kernel's form, scores and max pre-multiplied by
// sl2 (each product rounded once); out_raw[i]: the prefill kernel's form,
// one FMA of the raw score against the scaled max.
__global__ void softmax_weights_kernel(const float* __restrict__ s, const float* __restrict__ m,
                                       int64_t n, float sl2, float* __restrict__ out_scaled,
                                       float* __restrict__ out_raw) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    // The products are rounded on their own, as in the kernels (decode keeps
    // s*sl2 because it also feeds the row maximum, prefill scales the
    // maximum): written as one v_mul_f32 each so the compiler cannot contract
    // them into the subtraction, which would turn the decode form into the
    // prefill form.
    const float si = s[i];
    float m2, s2;
    asm volatile("v_mul_f32 %0, %1, %2" : "=v"(m2) : "v"(m[i]), "v"(sl2));
    asm volatile("v_mul_f32 %0, %1, %2" : "=v"(s2) : "v"(si), "v"(sl2));
    out_scaled[i] = qasr::softmax_w_scaled(s2, m2);
    out_raw[i] = qasr::softmax_w_raw(si, sl2, m2);
}

// ---- matrix-core calibration ------------------------------------------
// Each wave runs `mfma_iters` iterations of four independent
// v_mfma_f32_32x32x16_f16 chains (the prefill kernel's MFMA) and/or
// `valu_iters` iterations of a softmax-shaped VALU block over 16 values (the
// prefill kernel's per-score mix: a row max, one FMA and one v_exp_f32 per
// value, packed f16 conversion and a v_dot2 row sum).  MODE 0: every wave
// MFMA only; 1: every wave VALU only; 2: an 8-wave workgroup whose waves 0-3
// run the MFMA part and waves 4-7 the VALU part, i.e. one of each per SIMD;
// 3: every wave both, interleaved in one loop.  Wave 0 of workgroup 0
// records s_memtime (shader clock) and s_memrealtime (100 MHz) at its start
// and end in clk[0..3].
template <int MODE, int KIND>
__global__ void mfma_probe_kernel(int mfma_iters, int valu_iters, float* __restrict__ sink,
                                  unsigned long long* __restrict__ clk) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool do_mfma = MODE == 0 || MODE == 3 || (MODE == 2 && wave < 4);
    const bool do_valu = MODE == 1 || MODE == 3 || (MODE == 2 && wave >= 4);
    const bool timer = blockIdx.x == 0 && threadIdx.x == 0;
    unsigned long long t0 = 0, r0 = 0;
    if (timer) {
        t0 = __builtin_amdgcn_s_memtime();
        r0 = __builtin_amdgcn_s_memrealtime();
    }
    qasr::half8v a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (f16)(0.01f * lane + 0.125f * e);
        b[e] = (f16)(1.0f - 0.001f * lane * e);
    }
    qasr::float16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
    float v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0.001f * lane + 0.01f * i;
    float m = 0.5f, sum = 0.0f;
    const float sl2 = 0.1275f;
    const qasr::half2v ones = {(f16)1.0f, (f16)1.0f};
    auto mfma_block = [&]() {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
    };
    // KIND 0: the whole softmax mix; 1: only the exponentials (v_exp_f32 of
    // an FMA); 2: only FMAs; 3: only v_dot2 sums; 4: only packed f16
    // conversions; 5: only row maxima (v_max3); 6: the mix with the row sum
    // in f32 adds instead of v_dot2; 7: the mix with single conversions
    // (v_cvt_f16_f32) instead of packed ones.
    auto valu_block = [&](int it) {
        const float d = 1e-6f * (float)it;  // new scores each iteration
        if constexpr (KIND == 1) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = qasr::fast_exp2(fmaf(v[i], sl2, d));
        } else if constexpr (KIND == 2) {
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = fmaf(v[i], sl2, d);
        } else if constexpr (KIND == 3) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const qasr::half2v pk = {(f16)(0.5f * i), (f16)d};
                sum = __builtin_amdgcn_fdot2(pk, ones, sum, false);
            }
        } else if constexpr (KIND == 4) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const qasr::half2v pk = {(f16)(v[2 * i] + d), (f16)v[2 * i + 1]};
                v[2 * i + 1] = __builtin_bit_cast(float, pk);
            }
        } else if constexpr (KIND == 5) {
            float mx = kNegInfProbe;
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, v[i] + (i == 0 ? d : 0.0f));
            m = fmaxf(m, mx);
            v[0] = m;
        } else {
            float mx = kNegInfProbe;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                v[i] += d;
                mx = fmaxf(mx, v[i]);
            }
            m = fmaxf(m, mx * sl2);
            float e[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) e[i] = qasr::softmax_w_raw(v[i], sl2, m);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if constexpr (KIND == 6) {
                    const qasr::half2v pk = {(f16)e[2 * i], (f16)e[2 * i + 1]};
                    sum += (float)pk[0] + (float)pk[1];
                } else if constexpr (KIND == 7) {
                    f16 lo = (f16)e[2 * i], hi = (f16)e[2 * i + 1];
                    asm volatile("" : "+v"(lo), "+v"(hi));  // keep them single conversions
                    const qasr::half2v pk = {lo, hi};
                    sum = __builtin_amdgcn_fdot2(pk, ones, sum, false);
                } else {
                    const qasr::half2v pk = {(f16)e[2 * i], (f16)e[2 * i + 1]};
                    sum = __builtin_amdgcn_fdot2(pk, ones, sum, false);
                }
            }
        }
    };
    if constexpr (MODE == 3) {
        const int n = max(mfma_iters, valu_iters);
        for (int it = 0; it < n; ++it) {
            if (it < mfma_iters) mfma_block();
            if (it < valu_iters) valu_block(it);
        }
    } else {
        if (do_mfma)
            for (int it = 0; it < mfma_iters; ++it) mfma_block();
        if (do_valu)
            for (int it = 0; it < valu_iters; ++it) valu_block(it);
    }
    float acc = sum + m;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc += c0[i] + c1[i] + c2[i] + c3[i] + v[i];
    if (lane == 0) sink[blockIdx.x * (blockDim.x >> 6) + wave] = acc;
    if (timer) {
        clk[0] = t0;
        clk[1] = r0;
        clk[2] = __builtin_amdgcn_s_memtime();
        clk[3] = __builtin_amdgcn_s_memrealtime();
    }
}

}  // namespace

namespace {

template <int KIND>
void launch_probe(int mode, dim3 grid, dim3 block, hipStream_t st, int mi, int vi, float* sink,
                  unsigned long long* clk) {
    switch (mode) {
        case 0: hipLaunchKernelGGL((mfma_probe_kernel<0, KIND>), grid, block, 0, st, mi, vi, sink, clk); break;
        case 1: hipLaunchKernelGGL((mfma_probe_kernel<1, KIND>), grid, block, 0, st, mi, vi, sink, clk); break;
        case 2: hipLaunchKernelGGL((mfma_probe_kernel<2, KIND>), grid, block, 0, st, mi, vi, sink, clk); break;
        default: hipLaunchKernelGGL((mfma_probe_kernel<3, KIND>), grid, block, 0, st, mi, vi, sink, clk); break;
    }
}

}  // namespace

extern "C" int qasr_mfma_probe(qasr_ctx* ctx, int mode, int wgs, int waves, int mfma_iters,
                               int valu_iters, float* sink_dev, unsigned long long* clk_dev,
                               void* stream) {
    if (!ctx) return fail(QASR_EINVAL, "null context");
    if (!sink_dev || !clk_dev) return fail(QASR_EINVAL, "null device pointer");
    // mode = base mode (0..3) + 4 * VALU kind (0..7)
    if (mode < 0) return fail(QASR_EINVAL, "negative mode");
    const int kind = mode >> 2;
    mode &= 3;
    if (kind > 7) return fail(QASR_EINVAL, "VALU kind %d outside [0, 7]", kind);
    if (mode == 2) waves = 8;  // four MFMA and four VALU waves
    if (wgs <= 0 || wgs > 65536 || waves <= 0 || waves > 16 || mfma_iters < 0 || valu_iters < 0)
        return fail(QASR_EINVAL, "wgs in [1, 65536], waves in [1, 16], iterations >= 0");
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    const dim3 grid(wgs), block(waves * 64);
    const hipStream_t st = (hipStream_t)stream;
    switch (kind) {
        case 0: launch_probe<0>(mode, grid, block, st, mfma_iters, valu_iters, sink_dev, clk_dev); break;
        case 1: launch_probe<1>(mode, grid, block, st, mfma_iters, valu_iters, sink_dev, clk_dev); break;
        case 2: launch_probe<2>(mode, grid, block, st, mfma_iters, valu_iters, sink_dev, clk_dev); break;
        case 3: launch_probe<3>(mode, grid, block, st, mfma_iters, valu_iters, sink_dev, clk_dev); break;
        case 4: launch_probe<4>(mode, grid, block, st, mfma_iters, valu_iters, sink_dev, clk_dev); break;
        case 5: launch_probe<5>(mode, grid, block, st, mfma_iters, valu_iters, sink_dev, clk_dev); break;
        case 6: launch_probe<6>(mode, grid, block, st, mfma_iters, valu_iters, sink_dev, clk_dev); break;
        default: launch_probe<7>(mode, grid, block, st, mfma_iters, valu_iters, sink_dev, clk_dev); break;
    }
    HIP_TRY(hipGetLastError(), "mfma probe launch");
    return QASR_OK;
}

extern "C" int qasr_softmax_weights(qasr_ctx* ctx, const float* s_dev, const float* m_dev,
                                    int64_t n, float* out_scaled_dev, float* out_raw_dev,
                                    void* stream) {
    if (!ctx) return fail(QASR_EINVAL, "null context");
    if (n < 0) return fail(QASR_EINVAL, "negative n");
    if (n == 0) return QASR_OK;
    if (!s_dev || !m_dev || !out_scaled_dev || !out_raw_dev)
        return fail(QASR_EINVAL, "null device pointer");
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    const int threads = 256;
    const int64_t blocks = (n + threads - 1) / threads;
    if (blocks > 0x7fffffff) return fail(QASR_EINVAL, "n too large");
    hipLaunchKernelGGL(softmax_weights_kernel, dim3((unsigned)blocks), dim3(threads), 0,
                       (hipStream_t)stream, s_dev, m_dev, n, ctx->scale_log2, out_scaled_dev,
                       out_raw_dev);
    HIP_TRY(hipGetLastError(), "softmax weights launch");
    return QASR_OK;
}

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Bare streaming read: workgroup w reads bytes [w*per, (w+1)*per) of src with
// non-temporal dwordx4 buffer loads (the decode kernel's K/V load form), each
// wave holding `kDepth` loads per lane in flight, and folds them into one
// word so the loads are live; lane 0 of each wave writes its fold to sink.
constexpr int kDepth = 16;

__global__ void stream_read_kernel(const uint8_t* __restrict__ src, int64_t per,
                                   uint32_t* __restrict__ sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const uint8_t* base = src + (int64_t)blockIdx.x * per;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, (int)per, 0x00020000);
    const int step = waves * 1024;  // bytes per workgroup pass of one load per lane
    uint32_t acc = 0;
    for (int off = wave * 1024 + lane * 16; off < per; off += kDepth * step) {
        u32x4 v[kDepth];
#pragma unroll
        for (int k = 0; k < kDepth; ++k)
            v[k] = __builtin_amdgcn_raw_buffer_load_b128(r, off + k * step, 0, 2);
#pragma unroll
        for (int k = 0; k < kDepth; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    if (lane == 0) sink[blockIdx.x * waves + wave] = acc;
}

}  // namespace

extern "C" int qasr_stream_read(qasr_ctx* ctx, const void* src_dev, int64_t bytes, int wgs,
                                int waves, uint32_t* sink_dev, void* stream) {
    if (!ctx) return fail(QASR_EINVAL, "null context");
    if (!src_dev || !sink_dev) return fail(QASR_EINVAL, "null device pointer");
    if (wgs <= 0 || wgs > 65536 || waves <= 0 || waves > 16)
        return fail(QASR_EINVAL, "wgs in [1, 65536], waves in [1, 16]");
    if (bytes <= 0 || bytes % ((int64_t)wgs * 16) != 0)
        return fail(QASR_EINVAL, "bytes must be a positive multiple of 16 * wgs");
    const int64_t per = bytes / wgs;
    if (per > (1 << 30)) return fail(QASR_EINVAL, "more than 1 GiB per workgroup");
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    hipLaunchKernelGGL(stream_read_kernel, dim3(wgs), dim3(waves * 64), 0, (hipStream_t)stream,
                       (const uint8_t*)src_dev, per, sink_dev);
    HIP_TRY(hipGetLastError(), "stream read launch");
    return QASR_OK;
}
