// diag.hip -- qasr_softmax_weights: the attention kernels' softmax-weight
// exponent (common.hpp softmax_w_scaled / softmax_w_raw) evaluated over
// caller arrays, so tests can hold it against the reference's libm expf
// (cpu_decoder.rs:292-365 forms e = expf(s*scale - max*scale)).

#include "abi_internal.hpp"

using qasr::f16;
using qasr_abi::DeviceScope;
using qasr_abi::fail;
using qasr_abi::hip_fail;

namespace {

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

}  // namespace

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
