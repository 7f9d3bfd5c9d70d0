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

}  // namespace qasr
