// common.hpp -- shared device helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qasr {

constexpr int kHeadDim = 128;   // head_dim of both Qwen3-ASR decoders
constexpr int kRep = 2;         // q heads per kv head (16 / 8)
constexpr int kMaxBatch = 64;   // batch entries planned per launch (kernel-argument arrays)

typedef _Float16 f16;
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float h2f(f16 h) { return (float)h; }
// v_cvt_f16_f32 under the default mode register: round-to-nearest-even, f16
// subnormals kept -- the rounding of half::f16::from_f32.
__device__ __forceinline__ f16 f2h(float f) { return (f16)f; }

// 16 bytes = 8 halves, moved as one dwordx4.
union H8 {
    uint4 u;
    half8v h;
    half2v h2[4];
    f16 e[8];
};

// ---- direct global -> LDS copies ---------------------------------------
// A buffer resource as four dwords (for inline asm), `bytes` the range past
// which loads return zeros (and copies write nothing).
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4v make_rsrc_words(const void* p, int bytes) {
    const uint64_t a = (uint64_t)p;
    return (u32x4v){(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)bytes, 0x00020000u};
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// One `buffer_load_dwordx4 ... lds`: lane l's 16 bytes from byte offset voff
// of the resource land at LDS address lds + 16 l (M0 = lds).  Issued as
// inline asm, so the compiler does not wait for it before unrelated LDS
// reads; the caller waits for it itself (vmcnt) before reading its bytes.
__device__ __forceinline__ void dma16(u32x4v rsrc, int voff, uint32_t lds) {
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}
// The same copy as a device-coherent (sc1) load: it reads what other
// workgroups published with device-scope stores.
__device__ __forceinline__ void dma16_sc1(u32x4v rsrc, int voff, uint32_t lds) {
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen sc1 lds" ::"v"(voff), "s"(rsrc), "{m0}"(lds) : "memory");
}

// ---- DPP cross-lane moves inside a 16-lane row (no LDS traffic) ----------
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRor4 = 0x124;       // row_ror:4
constexpr int kDppRor8 = 0x128;       // row_ror:8
constexpr int kDppMirror = 0x140;     // row_mirror      (lane i <- 15-i)
constexpr int kDppHalfMirror = 0x141; // row_half_mirror (lane i <- 7-i in each half)

// Sum over the 16 lanes of a row; every lane of the row gets the total.
__device__ __forceinline__ float row_sum16(float x) {
    x += dpp<kDppXor1>(x);
    x += dpp<kDppXor2>(x);
    x += dpp<kDppHalfMirror>(x);
    x += dpp<kDppMirror>(x);
    return x;
}

// Transposing reduction of 16 values over a 16-lane row: lane i of the row
// ends with the row-wide sum of value index i.  Each step pairs the lane with
// a partner in the other half of the current index bit (row_mirror: bit 3,
// row_half_mirror: bit 2, quad_perm: bits 1 and 0), keeps the half of the
// values whose index bit equals its own lane bit and adds the partner's copy
// of them: 15 DPP adds and 30 selects instead of 64 DPP adds.
__device__ __forceinline__ float row_reduce_transpose16(const float (&v)[16], int i) {
    float w[8], x[4], y[2];
    const bool b3 = i & 8, b2 = i & 4, b1 = i & 2, b0 = i & 1;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float keep = b3 ? v[k + 8] : v[k], send = b3 ? v[k] : v[k + 8];
        w[k] = keep + dpp<kDppMirror>(send);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float keep = b2 ? w[k + 4] : w[k], send = b2 ? w[k] : w[k + 4];
        x[k] = keep + dpp<kDppHalfMirror>(send);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const float keep = b1 ? x[k + 2] : x[k], send = b1 ? x[k] : x[k + 2];
        y[k] = keep + dpp<kDppXor2>(send);
    }
    const float keep = b0 ? y[1] : y[0], send = b0 ? y[0] : y[1];
    return keep + dpp<kDppXor1>(send);
}

// acc += p * f16 (low / high half of a packed dword), one v_fma_mix_f32 with a
// single rounding (as fmaf(p, (float)h, acc)).  Written out so the packed
// register feeds both halves through op_sel instead of being unpacked into
// extra registers first.
__device__ __forceinline__ void fma_mix_lo(float& acc, float p, uint32_t pk) {
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(p), "v"(pk));
}
__device__ __forceinline__ void fma_mix_hi(float& acc, float p, uint32_t pk) {
    asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(p), "v"(pk));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Softmax weights in the exp2 domain.  The reference forms
// e = expf(s*scale - max*scale) (cpu_decoder.rs:292-365); the kernels fold
// log2(e) into the scale (sl2 = scale*log2(e), rounded once on the host) and
// exponentiate with v_exp_f32:
//  - decode keeps scores pre-multiplied (s2 = s*sl2) and its running max in
//    that domain (m2): w = 2^(s2 - m2);
//  - prefill keeps raw scores and folds the multiply into one FMA against
//    the scaled max: w = 2^(fma(s, sl2, -m2)).
// qasr_softmax_weights evaluates both forms for the tests against glibc expf.
__device__ __forceinline__ float softmax_w_scaled(float s2, float m2) { return fast_exp2(s2 - m2); }
__device__ __forceinline__ float softmax_w_raw(float s, float sl2, float m2) {
    return fast_exp2(fmaf(s, sl2, -m2));
}

// ---- publishing partial results to other workgroups ---------------------
// MI355X has one L2 per XCD and they are not coherent with each other inside
// a kernel.  An agent-scope release/acquire fence would write back and
// invalidate the whole L2 (buffer_wbl2 / buffer_inv) in every workgroup, so
// split-K partials are instead moved with device-scope ("sc1") accesses only:
// relaxed agent-scope atomic stores write through to the device-coherent
// level, relaxed agent-scope atomic loads miss in the non-coherent caches.
// The writer waits for its stores to complete (vmcnt(0)) before the
// workgroup bumps the arrival ticket; the reader issues its loads only after
// the ticket says every partial has arrived.
__device__ __forceinline__ void store_dev(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_dev(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// All of this wave's memory operations complete, then a workgroup barrier.
__device__ __forceinline__ void stores_done_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt/lgkmcnt unconstrained
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
}
__device__ __forceinline__ uint32_t ticket_add(uint32_t* p) {
    return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Arrival of n partials at once; returns the count before them.
__device__ __forceinline__ uint32_t ticket_add_n(uint32_t* p, uint32_t n) {
    return __hip_atomic_fetch_add(p, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ticket_reset(uint32_t* p) {
    __hip_atomic_store(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace qasr
