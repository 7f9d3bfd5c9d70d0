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

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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
__device__ __forceinline__ void ticket_reset(uint32_t* p) {
    __hip_atomic_store(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace qasr
