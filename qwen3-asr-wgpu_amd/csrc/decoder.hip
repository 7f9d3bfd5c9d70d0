// decoder.hip -- the whole Qwen3 text decoder around the attention path: the
// C ABI's qasr_decoder_* (include/qasr_attn.h).
//
// Layer sequence and rounding points of the reference's CpuTextDecoder
// (src/cpu_decoder.rs:367-532), which WgpuTextDecoder::step / ::prefill run
// on the GPU (src/decoder.rs:1768-1925, 4489-5244):
//   n  = f16(rms_norm(x) * input_norm)                    cpu_decoder.rs:261-271, 386-389
//   qkv = f16(n . W_qkv^T)                                 398-400
//   stage (a) + (b) [decode] or (a) + (c) [prefill]       this library
//   x  = f16(x + attn . W_o^T)                             431 (batch_dot_acc, 45-62)
//   n2 = f16(rms_norm(x) * post_norm)                      435-438
//   g|u = f16(n2 . W_gate_up^T)                            440-441
//   h  = f16(g / (1 + exp(-g)) * u)                        442-448
//   x  = f16(x + h . W_down^T)                             449
// then logits = f32(rms_norm(x_last) * norm . E^T) against the tied embedding
// and the first maximal index (458-485).
//
// The projections of a decode step run this file's skinny MFMA kernels; the
// prefill projections are plain GEMMs and run gemm.hip's MFMA kernel (f16
// operands, f32 accumulation, one f16 rounding of the f32 result; with a
// residual, x + dot is rounded once as in batch_dot_acc).  Its summation order
// does not depend on the row count, so a prompt prefilled alone and inside a
// batch gives the same bits (the library's stream-K kernels split K by the
// row count).  QASR_PREFILL_GEMM=blas sends them to rocBLAS instead (beta = 1
// for the residual; measured 1.4-2.5x faster at these shapes, not row
// invariant).  The elementwise steps are small HIP kernels below.  Nothing here allocates per
// call: the activation workspace is sized for max_rows at creation, and
// rocBLAS gets a fixed workspace so that a step can be captured in a graph.

#include <rocblas/rocblas.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <string>
#include <vector>

#include "abi_internal.hpp"
#include "common.hpp"

using qasr::f16;
using qasr::H8;
using qasr_abi::DeviceScope;
using qasr_abi::fail;
using qasr_abi::hip_fail;

namespace {

constexpr int kNormThreads = 256;
constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxChunks = 32;  // workgroups per logits row in the first argmax pass
constexpr int kHeadRows = 16;      // rows per logits GEMM + argmax: one skinny launch (kSkinnyRows)
constexpr size_t kBlasWorkspace = size_t(64) << 20;
constexpr int kMaxPrefillSegs = 64;  // segments of one batched prefill call
// Rows of one call (decode batch or prefill): bounds the activation
// workspace (about 61 KB per row at the 1.7B shape, 1 GB at the limit).
constexpr int kMaxDecoderRows = 16384;

// ---- block reductions (wave64 shuffles, then one LDS pass) ---------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

// N independent wave_sums, each step's N exchanges issued together (one LDS
// latency per step instead of one per value).  Each lane adds the same pairs
// as wave_sum, so every result is bit-identical to wave_sum's.
template <int N>
__device__ __forceinline__ void wave_sums(float (&v)[N]) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        float o[N];
#pragma unroll
        for (int i = 0; i < N; ++i) o[i] = __shfl_xor(v[i], m);
#pragma unroll
        for (int i = 0; i < N; ++i) v[i] += o[i];
    }
}

// (value, index) pair order for the argmax: larger value, then smaller index
// (the reference keeps the first maximal index: `if v > logits[best]`).
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(v, m);
        const int oi = __shfl_xor(i, m);
        if (better(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    }
}

// ---- kernels -------------------------------------------------------------

// Embedding rows of the batch's tokens (embed_row, cpu_decoder.rs:255-258).
// An id outside [0, vocab) reads row 0 (the caller's contract says in range).
// With ss set (hs <= 2048, one 8-element chunk per thread), also each chunk's
// sum of squares, fmaf from 0 in element order: the chunk sums a fused
// RMSNorm of the first projection starts from (ss[r][c], 256 per row).
__global__ __launch_bounds__(256) void embed_rows_kernel(const f16* __restrict__ embed,
                                                         const int32_t* __restrict__ tokens,
                                                         int vocab, int hs, f16* __restrict__ x,
                                                         float* __restrict__ ss) {
    const int r = blockIdx.x;
    int t = tokens[r];
    if (t < 0 || t >= vocab) t = 0;
    const uint4* src = (const uint4*)(embed + (int64_t)t * hs);
    uint4* dst = (uint4*)(x + (int64_t)r * hs);
    for (int c = threadIdx.x; c < hs / 8; c += blockDim.x) {
        H8 v;
        v.u = src[c];
        dst[c] = v.u;
        if (ss) {
            float a = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float f = (float)v.e[e];
                a = fmaf(f, f, a);
            }
            ss[r * 256 + c] = a;
        }
    }
}

// The last row of every segment of a batched prefill, packed: dst[r] =
// src[rows.idx[r]] (rows of hs f16; hs a multiple of 8).
struct RowList {
    int32_t idx[kMaxPrefillSegs];
};

__global__ __launch_bounds__(256) void gather_rows_kernel(const f16* __restrict__ src, int hs,
                                                          RowList rows, f16* __restrict__ dst) {
    const int r = blockIdx.x;
    const uint4* from = (const uint4*)(src + (int64_t)rows.idx[r] * hs);
    uint4* to = (uint4*)(dst + (int64_t)r * hs);
    for (int c = threadIdx.x; c < hs / 8; c += blockDim.x) to[c] = from[c];
}

// out[r] = f16((x * inv) * w) with inv = 1 / sqrt(sum(x^2) / n + eps), f32
// (rms_norm_row, cpu_decoder.rs:261-271).  One workgroup per row; the sum of
// squares is a tree sum (the reference sums in index order, so inv can
// differ from it in the last bit).
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const f16* __restrict__ x,
                                                                int64_t x_stride,
                                                                const f16* __restrict__ w,
                                                                f16* __restrict__ out, int n,
                                                                float eps) {
    __shared__ float s_part[kNormThreads / 64];
    const f16* xr = x + (int64_t)blockIdx.x * x_stride;
    f16* orow = out + (int64_t)blockIdx.x * n;
    float s = 0.0f;
    for (int c = threadIdx.x; c < n / 8; c += kNormThreads) {
        H8 v;
        v.u = ((const uint4*)xr)[c];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float f = (float)v.e[e];
            s = fmaf(f, f, s);
        }
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormThreads / 64; ++i) tot += s_part[i];
    const float inv = 1.0f / sqrtf(tot / (float)n + eps);
    for (int c = threadIdx.x; c < n / 8; c += kNormThreads) {
        H8 v, g, o;
        v.u = ((const uint4*)xr)[c];
        g.u = ((const uint4*)w)[c];
#pragma unroll
        for (int e = 0; e < 8; ++e) o.e[e] = (f16)(((float)v.e[e] * inv) * (float)g.e[e]);
        ((uint4*)orow)[c] = o.u;
    }
}

// h[r][i] = f16(g / (1 + exp(-g)) * u), g|u = gu[r][i], gu[r][inter + i]
// (cpu_decoder.rs:442-448).  8 elements per thread.
// f16(x) of an f32 value that is first rounded to f32: the reference's
// f16::from_f32 of an f32 result.  Without the register barrier the compiler
// folds the product or fma producing x into v_fma_mixlo_f16, which rounds the
// exact result once, straight to f16, and differs from f16(f32(.)) on about
// 2 in 10^5 products (measured on gfx950).
__device__ __forceinline__ f16 f16_of_f32(float x) {
    asm volatile("" : "+v"(x));
    return (f16)x;
}

// SiLU(g) * u in f32 (silu, cpu_decoder.rs): g / (1 + e^-g), then times u.
__device__ __forceinline__ float silu_times(float g, float u) {
    return g / (1.0f + expf(-g)) * u;
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const f16* __restrict__ gu, int inter,
                                                       int rows, f16* __restrict__ h) {
    const int per_row = inter / 8;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * per_row) return;
    const int r = (int)(idx / per_row), c = (int)(idx - (int64_t)r * per_row);
    const f16* grow = gu + (int64_t)r * 2 * inter;
    H8 g, u, o;
    g.u = ((const uint4*)grow)[c];
    u.u = ((const uint4*)(grow + inter))[c];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        o.e[e] = f16_of_f32(silu_times((float)g.e[e], (float)u.e[e]));
    }
    ((uint4*)(h + (int64_t)r * inter))[c] = o.u;
}

// First argmax pass: workgroup (chunk, row) finds the best (value, index) of
// its contiguous chunk of the row.
__global__ __launch_bounds__(kArgmaxThreads) void argmax_partial_kernel(
    const float* __restrict__ logits, int vocab, float* __restrict__ pv, int* __restrict__ pi) {
    __shared__ float s_v[kArgmaxThreads / 64];
    __shared__ int s_i[kArgmaxThreads / 64];
    const int row = blockIdx.y, chunk = blockIdx.x;
    const int per = (vocab + kArgmaxChunks - 1) / kArgmaxChunks;
    const int lo = chunk * per, hi = min(vocab, lo + per);
    const float* lr = logits + (int64_t)row * vocab;
    float bv = -__builtin_inff();
    int bi = vocab;  // no candidate yet
    for (int i = lo + threadIdx.x; i < hi; i += kArgmaxThreads) {
        const float v = lr[i];
        if (better(v, i, bv, bi)) {
            bv = v;
            bi = i;
        }
    }
    wave_argmax(bv, bi);
    if ((threadIdx.x & 63) == 0) {
        s_v[threadIdx.x >> 6] = bv;
        s_i[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgmaxThreads / 64; ++w)
            if (better(s_v[w], s_i[w], bv, bi)) {
                bv = s_v[w];
                bi = s_i[w];
            }
        pv[row * kArgmaxChunks + chunk] = bv;
        pi[row * kArgmaxChunks + chunk] = bi;
    }
}

// Second pass: one wave per row over the chunks' candidates.  A row whose
// values are all NaN (no candidate) yields 0, as the reference's loop does.
__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ pv,
                                                          const int* __restrict__ pi, int vocab,
                                                          int32_t* __restrict__ out) {
    const int row = blockIdx.x, lane = threadIdx.x;
    float bv = -__builtin_inff();
    int bi = vocab;
    if (lane < kArgmaxChunks) {
        bv = pv[row * kArgmaxChunks + lane];
        bi = pi[row * kArgmaxChunks + lane];
    }
    wave_argmax(bv, bi);
    if (lane == 0) out[row] = bi < vocab ? bi : 0;
}

// The argmax over the skinny logits kernel's per-tile candidates (one
// workgroup per row): the same (value, index) order, so the same token as the
// two passes over the logits.
constexpr int kArgTilesThreads = 1024;
constexpr int kArgTilesUnroll = 10;  // 10,240 candidates per round: the 151,936-entry vocabulary's 9,496 tiles
__global__ __launch_bounds__(kArgTilesThreads) void argmax_tiles_kernel(const float* __restrict__ pv,
                                                                        const int* __restrict__ pi,
                                                                        int ntiles, int vocab,
                                                                        int32_t* __restrict__ out) {
    __shared__ float s_v[kArgTilesThreads / 64];
    __shared__ int s_i[kArgTilesThreads / 64];
    const int row = blockIdx.x;
    const float* rv = pv + (int64_t)row * ntiles;
    const int* ri = pi + (int64_t)row * ntiles;
    float bv = -__builtin_inff();
    int bi = vocab;
    for (int base = 0; base < ntiles; base += kArgTilesThreads * kArgTilesUnroll) {
        // Every load of the round is issued before the first compare.
        float v[kArgTilesUnroll];
        int ix[kArgTilesUnroll];
#pragma unroll
        for (int u = 0; u < kArgTilesUnroll; ++u) {
            const int t = base + u * kArgTilesThreads + (int)threadIdx.x;
            v[u] = t < ntiles ? rv[t] : -__builtin_inff();
            ix[u] = t < ntiles ? ri[t] : vocab;
        }
#pragma unroll
        for (int u = 0; u < kArgTilesUnroll; ++u)
            if (better(v[u], ix[u], bv, bi)) {
                bv = v[u];
                bi = ix[u];
            }
    }
    wave_argmax(bv, bi);
    if ((threadIdx.x & 63) == 0) {
        s_v[threadIdx.x >> 6] = bv;
        s_i[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kArgTilesThreads / 64; ++w)
            if (better(s_v[w], s_i[w], bv, bi)) {
                bv = s_v[w];
                bi = s_i[w];
            }
        out[row] = bi < vocab ? bi : 0;
    }
}

// ---- skinny GEMM: the projections of a decode step ----------------------
// Y[m][n] = X[m][k] . W[n][k]^T over at most 16 activation rows: a weight
// stream, HBM-bound, so each weight byte is read once and fed to
// v_mfma_f32_16x16x32_f16 straight from the load (no LDS staging).  The 16
// activation rows are the MFMA's A operand (lane l: row l%16, k 8*(l/16)..+8;
// rows >= M read zeros through the buffer range), 16 weight rows its B
// operand (lane l: W row n0 + l%16, the same k), and lane l holds
// D[4*(l/16) + i][l%16].  Workgroup (tile, group) = 16 output columns x one
// of `groups` K ranges; its KS waves take one K slice each, two stages of 4
// k-steps (16 x 1 KiB loads) in flight, and are summed in wave order.  With
// groups > 1 (projections with few column tiles, so that a launch still has
// ~512 workgroups) each workgroup publishes its 16 x 16 partial with
// device-coherent stores and the last of the tile's workgroups to arrive
// (ticket) sums the partials in group order: deterministic, no second launch.
// The result is rounded once -- with the residual y added in f32 first
// (kOutAcc), or kept f32 (kOutF32, logits).  kOutGlu is gate|up followed by
// SiLU(gate) * up: tile t takes gate rows 8t..8t+7 and up rows
// N/2+8t..N/2+8t+7 (lanes r and r+8 hold gate and up of one column), rounds
// both to f16 like the projection, and writes h = f16(SiLU(g) u) to column
// 8t + r of Y[m][N/2] -- the same values silu_mul_kernel makes from the
// gate|up rows.
constexpr int kOutF16 = 0, kOutAcc = 1, kOutF32 = 2, kOutGlu = 3;
constexpr int kSkinnyRows = 16;
constexpr int kSharedMinRows = 8;  // fewer rows: their loads are mostly out of range, nothing to share
// Fused RMSNorm in front of a skinny projection: hidden sizes up to 8 x this
// (one 8-element chunk per thread of rms_norm_kernel's 256).
constexpr int kNormMaxChunks = 256;
constexpr int kNormMaxK = 8 * kNormMaxChunks;
constexpr int kSkinnyUnroll = 4;                     // k-steps per stage (8 measured no faster)
constexpr int kSkinnyPair = 2 * 32 * kSkinnyUnroll;  // K per wave: a multiple (even stage count)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kSc1 = 16;              // buffer cache policy: device-coherent (sc1)
constexpr int kSkinnyMaxTiles = 512;  // column tiles of a split (groups > 1) projection
constexpr int kSkinnyMaxGroups = 12;
constexpr int kSkinnyTargetWgs = 512;
constexpr int kSkinnySplitWgs = 256;    // a split projection: one workgroup per CU
constexpr int kSkinnySplitMinK = 3072;  // shortest K cut across workgroups

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                             (int)std::min<int64_t>(bytes, 0x7fffffff), 0x00020000);
}

__device__ __forceinline__ qasr::half8v load8(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(qasr::half8v, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// One int8 weight row segment (8 values, two dwords) as the f16 values the
// reference's W8 kernels use: f16(q * s) with q * s rounded to f32 once.
// Each byte is offset by 128 (xor 0x80) so v_cvt_f32_ubyte reads q + 128
// exactly, and fma((q + 128), s, -128 s) = q s before its single rounding.
__device__ __forceinline__ qasr::half8v dequant8(uint32_t lo, uint32_t hi, float s) {
    qasr::half8v h;
    const uint32_t d[2] = {lo, hi};
#pragma unroll
    for (int w = 0; w < 2; ++w)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float q = (float)(int8_t)(d[w] >> (8 * j));  // exact
            h[4 * w + j] = f16_of_f32(q * s);
        }
    return h;
}

// Prefill-side int8 projections: the layer's weights dequantized once into a
// scratch f16 matrix for the GEMM, out[n][k] = f16(q[n][k] * scale[n]).
__global__ __launch_bounds__(256) void dequant_rows_kernel(const int8_t* __restrict__ q,
                                                           const float* __restrict__ scale,
                                                           int64_t n_rows, int k,
                                                           f16* __restrict__ out) {
    const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;  // 8 weights
    if (i >= n_rows * k) return;
    const float s = scale[i / k];
    const uint2 v = *(const uint2*)(q + i);
    *(qasr::half8v*)(out + i) = dequant8(v.x, v.y, s);
}

struct SkinnyArgs {
    const void* W;        // [N][K] f16, or int8 when `scale` is set
    const float* scale;   // int8 weights: [N] per-row scales
    const f16* X;  // [M][K]
    void* Y;       // [M][N] f16, or f32 logits (null: am_v / am_i only)
    int M, N, K, groups;
    float* ws;           // split partials
    uint32_t* counters;  // split tickets
    const f16* nw;       // fused RMSNorm: gain [K] (X is the raw residual stream)
    float eps;
    const float* ss_in;  // fused RMSNorm: X's chunk sums of squares [kSkinnyRows][kNormMaxChunks]
    float* ss_out;       // kOutAcc: write the result rows' chunk sums there (or null)
    float* am_v;         // kOutF32: each row's best (value, index) per column tile,
    int* am_i;           //   [M][N / 16], for argmax_tiles_kernel (or null)
};

// Fused RMSNorm prologue, in two halves so that its loads are issued ahead
// of the weight stream and are not queued behind it: issue() loads this
// thread's gain chunk and its share of the rows' chunk sums of squares
// ss[row][c] (the squares of elements 8c..8c+7 summed with fmaf from 0 in
// element order, written by the producer of X); finish() stages the gains as
// f32 in LDS and returns the inverse RMS of activation row r (this lane's
// row): 64 chunks at a time through the same wave64 butterfly, then the four
// partials added in order, as rms_norm_kernel does -- its thread t sums
// exactly chunk t when K <= 8 * 256 -- so the normed values match that
// kernel's bit for bit.  Rows >= M get 0 (their activations read as zeros).
template <int KS>
struct NormPrologue {
    static constexpr int kPairs = kSkinnyRows * 4;  // (row, group of 64 chunks): q = 4 row + group
    static constexpr int kPer = (kPairs + KS - 1) / KS;  // wave w takes q = w, w + KS, ..
    static_assert(KS * 64 >= kNormMaxChunks, "one gain chunk per thread");
    H8 gain;
    float v[kPer];

    __device__ void issue(const SkinnyArgs& p, int wave, int lane) {
        const int nch = p.K / 8;
        const int c = threadIdx.x;
        gain.u = c < nch ? *(const uint4*)(p.nw + 8 * c) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int q = wave + i * KS, row = q >> 2, ch = 64 * (q & 3) + lane;
            v[i] = (q < kPairs && row < p.M && ch < nch) ? p.ss_in[row * kNormMaxChunks + ch] : 0.0f;
        }
    }

    __device__ float finish(const SkinnyArgs& p, float* s_gain, float* s_part, int wave, int lane,
                            int r) {
        const int c = threadIdx.x;
        if (c < p.K / 8) {
            *(float4*)&s_gain[8 * c] =
                make_float4((float)gain.e[0], (float)gain.e[1], (float)gain.e[2], (float)gain.e[3]);
            *(float4*)&s_gain[8 * c + 4] =
                make_float4((float)gain.e[4], (float)gain.e[5], (float)gain.e[6], (float)gain.e[7]);
        }
        wave_sums(v);
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int q = wave + i * KS;
            if (lane == 0 && q < kPairs) s_part[q] = v[i];
        }
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) tot += s_part[r * 4 + i];
        return r < p.M ? 1.0f / sqrtf(tot / (float)p.K + p.eps) : 0.0f;
    }
};

// A finished 16 x 16 output tile (column tile `tile`): lane l holds
// D[4(l/16) + i][l%16], i < 4, in `sum`, summed over this workgroup's K range.
// With K groups, the group partials are published and the last of the tile's
// workgroups to arrive (ticket) sums them in group order.  Then the outputs
// per OUT (see skinny_gemm_kernel), and for kOutAcc with ss_out the result
// rows' chunk sums of squares.  s_y: 256 floats of this wave's LDS.
template <int OUT>
__device__ __forceinline__ void skinny_tile_out(const SkinnyArgs& p, qasr::float4v sum, int tile,
                                                int group, int lane, float* s_y,
                                                const f16* y_pre = nullptr) {
    const int r = lane & 15, g = lane >> 4;
    const int M = p.M, N = p.N, groups = p.groups;
    const int n0 = tile * 16;
    constexpr bool kGlu = OUT == kOutGlu;
    if (groups > 1) {
        // This wave's stores complete (vmcnt(0)) before the ticket, and the
        // last arrival reads every group's partial with device-coherent
        // loads.
        float* mine = p.ws + ((int64_t)tile * groups + group) * 256 + lane * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) qasr::store_dev(&mine[i], sum[i]);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        uint32_t old = 0;
        if (lane == 0) old = qasr::ticket_add(&p.counters[tile]);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old != (uint32_t)(groups - 1)) return;
        const __amdgpu_buffer_rsrc_t pres = rsrc(p.ws + (int64_t)tile * groups * 256, (int64_t)groups * 1024);
        sum = qasr::float4v{0.0f, 0.0f, 0.0f, 0.0f};
        for (int grp = 0; grp < groups; ++grp)
            sum += __builtin_bit_cast(qasr::float4v, __builtin_amdgcn_raw_buffer_load_b128(
                                                         pres, (grp * 64 + lane) * 16, 0, kSc1));
        if (lane == 0) qasr::ticket_reset(&p.counters[tile]);
    }
    const int n = n0 + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * g + i;
        if constexpr (kGlu) {
            // Lanes r and r^8 (same rows) exchange gate and up; every lane of
            // the wave takes part in the shuffle.
            const float v = (float)(f16)sum[i];
            const float up = __shfl_xor(v, 8);
            if (r < 8 && m < M)
                ((f16*)p.Y)[(int64_t)m * (N / 2) + 8 * tile + r] = f16_of_f32(silu_times(v, up));
            continue;
        }
        if (m >= M) continue;
        const int64_t idx = (int64_t)m * N + n;
        if constexpr (OUT == kOutF32) {
            if (p.Y) ((float*)p.Y)[idx] = sum[i];  // null: only the argmax candidates
        } else {
            f16* y = (f16*)p.Y;
            const f16 yv = OUT == kOutAcc ? (y_pre ? y_pre[i] : y[idx]) : (f16)0.0f;
            const f16 out = (f16)(OUT == kOutAcc ? (float)yv + sum[i] : sum[i]);
            y[idx] = out;
            if constexpr (OUT == kOutAcc) sum[i] = (float)out;  // for the chunk sums below
        }
    }
    if constexpr (OUT == kOutF32) {
        if (p.am_v) {
            // This tile's best (value, index) of each row, the argmax's first
            // pass without re-reading the logits: the 16 lanes of a row group
            // hold its 16 columns.  A NaN never becomes a candidate.
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float bv = -__builtin_inff();
                int bi = N;
                if (better(sum[i], n, bv, bi)) {
                    bv = sum[i];
                    bi = n;
                }
#pragma unroll
                for (int msk = 8; msk >= 1; msk >>= 1) {
                    const float ov = __shfl_xor(bv, msk);
                    const int oi = __shfl_xor(bi, msk);
                    if (better(ov, oi, bv, bi)) {
                        bv = ov;
                        bi = oi;
                    }
                }
                const int m = 4 * g + i;
                if (r == 0 && m < M) {
                    p.am_v[(int64_t)m * (N / 16) + tile] = bv;
                    p.am_i[(int64_t)m * (N / 16) + tile] = bi;
                }
            }
        }
    }
    if constexpr (OUT == kOutAcc) {
        if (p.ss_out) {
            // The next projection's half of a fused RMSNorm: this tile's two
            // 8-column chunks of every result row, squares summed with fmaf
            // in column order (rms_norm_kernel's per-thread sum), via this
            // wave's LDS scratch s_y ([16 rows][16 columns]).
#pragma unroll
            for (int i = 0; i < 4; ++i) s_y[(4 * g + i) * 16 + r] = sum[i];
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            __builtin_amdgcn_wave_barrier();
            const int row = lane >> 1, ch = lane & 1;
            if (lane < 32 && row < M) {
                float ss = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float f = s_y[row * 16 + 8 * ch + e];
                    ss = fmaf(f, f, ss);
                }
                p.ss_out[row * kNormMaxChunks + 2 * tile + ch] = ss;
            }
        }
    }
}

template <int KS, int U, bool W8, int OUT, bool NORM>
__global__ __launch_bounds__(KS * 64) void skinny_gemm_kernel(SkinnyArgs p) {
    __shared__ qasr::float4v s_red[KS][64];
    __shared__ __attribute__((aligned(16))) float s_gain[NORM ? kNormMaxK : 1];
    __shared__ float s_part[NORM ? kSkinnyRows * 4 : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int M = p.M, N = p.N, K = p.K, groups = p.groups;
    const int tile = blockIdx.x, n0 = tile * 16;
    const int kw = K / (KS * groups);
    const int kbeg = (blockIdx.y * KS + wave) * kw;
    constexpr int wbytes = W8 ? 1 : 2;  // bytes per weight
    // This lane's weight row: n0 + r, or for kOutGlu gate row 8t + r (r < 8)
    // and up row N/2 + 8t + r - 8, as an offset rr from the resource's first
    // row w0.
    constexpr bool kGlu = OUT == kOutGlu;
    const int w0 = kGlu ? 8 * tile : n0;
    const int rr = kGlu ? (r < 8 ? r : N / 2 + r - 8) : r;
    const int64_t wrows = kGlu ? (int64_t)(N / 2 + 8) : 16;
    const __amdgpu_buffer_rsrc_t wres =
        rsrc((const char*)p.W + (int64_t)w0 * K * wbytes, wrows * K * wbytes);
    float ws = 0.0f;  // W8: this lane's row's scale
    if constexpr (W8) {
        ws = p.scale[w0 + rr];
    }
    const __amdgpu_buffer_rsrc_t xres = rsrc(p.X, (int64_t)M * K * 2);
    const int woff = rr * K * 2 + g * 16;  // bytes: weight row rr, k 8g
    const int xoff = r * K * 2 + g * 16;   // bytes: activation row r, k 8g

    // Stages of U k-steps, double buffered: stage st+1's loads
    // are issued before stage st's MFMAs.
    struct Stage {
        qasr::half8v b[U], x[U];
        uint2 q[U];  // W8: the raw int8 weights
    };
    const int nst = kw / (32 * U);
    auto load_stage = [&](int st, Stage& S) {
        const int k0 = kbeg + st * 32 * U;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kk = k0 + 32 * u;
            if constexpr (W8) {
                S.q[u] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                       wres, rr * K + g * 8 + kk, 0, 0));
            } else {
                S.b[u] = load8(wres, woff + kk * 2);
            }
            S.x[u] = load8(xres, xoff + kk * 2);
        }
    };
    qasr::float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
    float inv = 0.0f;  // NORM: inverse RMS of activation row r
    // NORM: the activations are normed on the way into the MFMA, as
    // rms_norm_kernel rounds them: f16((x * inv) * gain).
    auto act = [&](const qasr::half8v& x, int kk) {
        if constexpr (NORM) {
            const float4 g0 = *(const float4*)&s_gain[kk + 8 * g];
            const float4 g1 = *(const float4*)&s_gain[kk + 8 * g + 4];
            const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
            qasr::half8v n;
#pragma unroll
            for (int e = 0; e < 8; ++e) n[e] = f16_of_f32(((float)x[e] * inv) * gv[e]);
            return n;
        } else {
            return x;
        }
    };
    auto mma_stage = [&](const Stage& S, int st) {
        const int k0 = kbeg + st * 32 * U;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const qasr::half8v xa = act(S.x[u], k0 + 32 * u);
            if constexpr (W8) {
                const qasr::half8v b = dequant8(S.q[u].x, S.q[u].y, ws);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, b, acc, 0, 0, 0);
            } else {
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, S.b[u], acc, 0, 0, 0);
            }
        }
    };
    // nst is even (the wave's K slice is a multiple of 64 U): stages 0 and 1
    // are requested first (after the fused norm's own loads), then each
    // stage's buffer is refilled two stages ahead as soon as its MFMAs are
    // issued, so two stages are always in flight -- the norm prologue too
    // runs under them.
    Stage s0, s1;
    NormPrologue<KS> np;
    if constexpr (NORM) np.issue(p, wave, lane);
    // The residual this lane's outputs add (rows 4 g + i, column n0 + r),
    // requested ahead of the weight stream so the epilogue does not wait a
    // memory round trip for it (nothing in this launch writes it before the
    // epilogue reads it).
    f16 y_pre[4] = {};
    if constexpr (OUT == kOutAcc) {
        if (wave == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (4 * g + i < M) y_pre[i] = ((const f16*)p.Y)[(int64_t)(4 * g + i) * N + n0 + r];
        }
    }
    // With 8 or more rows the second stage is requested after the folded
    // norm's inputs have arrived: requested together, they queued behind the
    // weight stages (16-slot step 1838 -> 1813 us).  One row keeps both
    // stages first (0.6B one-slot step 964 against 967 us).
    const bool norm_first = NORM && M >= kSharedMinRows;
    load_stage(0, s0);
    if (norm_first) inv = np.finish(p, s_gain, s_part, wave, lane, r);
    load_stage(1, s1);
    if (NORM && !norm_first) inv = np.finish(p, s_gain, s_part, wave, lane, r);
    int st = 0;
    for (; st + 2 < nst; st += 2) {
        __builtin_amdgcn_sched_barrier(0);
        mma_stage(s0, st);
        __builtin_amdgcn_sched_barrier(0);
        load_stage(st + 2, s0);
        __builtin_amdgcn_sched_barrier(0);
        mma_stage(s1, st + 1);
        __builtin_amdgcn_sched_barrier(0);
        load_stage(st + 3, s1);
    }
    __builtin_amdgcn_sched_barrier(0);
    mma_stage(s0, st);
    __builtin_amdgcn_sched_barrier(0);
    mma_stage(s1, st + 1);
    s_red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    qasr::float4v sum = s_red[0][lane];
#pragma unroll
    for (int w = 1; w < KS; ++w) sum += s_red[w][lane];
    skinny_tile_out<OUT>(p, sum, tile, blockIdx.y, lane, reinterpret_cast<float*>(&s_red[0][0]),
                         OUT == kOutAcc ? y_pre : nullptr);
}

// ---- skinny GEMM with the weight rows staged in LDS ------------------------
// The same product as skinny_gemm_kernel, for very wide outputs: a workgroup
// is 4 waves over `tpw` consecutive column tiles of one K group, and wave w
// takes K range [(group*4 + w) kw, +kw), kw = 32 NKS.  The wave loads its
// activation slice once, into registers (normed there once when NORM), and
// uses it for all its tiles -- skinny_gemm_kernel reloads it with every
// k-step of every tile, as many bytes as the weights at 16 rows.  Each tile's
// 16 row slices stream by direct global->LDS copies (1024 / RB rows per copy
// instruction, every row slice one contiguous run) into the wave's own LDS
// buffer -- NBUF of them, so tile t+2 streams while t+1 is next -- and the
// MFMA B operand is read back from LDS.  No wave reads another's buffer, so
// the stream needs no barrier; each wave leaves its per-tile partial in LDS,
// and after the last tile wave w finishes tiles w, w+4, .. (the four partials
// summed in wave order, then skinny_tile_out).  Copies are waited for by
// count (they are inline asm); the epilogues' stores come after the last
// copy.  LDS row slice layout: 16-byte chunk c of row n at slot c ^ n, so
// the operand read (16 rows at one k) is conflict-free.
constexpr int kLdsWaves = 4;
constexpr int kLdsMaxTiles = 4;     // column tiles per workgroup
constexpr int kLdsMinTiles = 2048;  // outputs at least this wide ..
constexpr int kLdsMinRows = 8;      // .. of at least this many rows take the kernel

template <int NKS, bool W8, int OUT, bool NORM, int NBUF>
__global__ __launch_bounds__(kLdsWaves * 64) void skinny_lds_kernel(SkinnyArgs p, int tpw) {
    constexpr int wbytes = W8 ? 1 : 2;
    constexpr int KW = 32 * NKS;     // K per wave
    constexpr int RB = KW * wbytes;  // bytes of one row slice
    static_assert(RB >= 256 && RB <= 1024, "row slices of 256..1024 bytes");
    constexpr int LPR = RB / 16;   // copy lanes per row, 16..64
    constexpr int RPI = 64 / LPR;  // rows per copy instruction, 1..4
    constexpr int NCP = 16 / RPI;  // copy instructions per tile and wave
    constexpr int TB = 16 * RB;    // one wave's tile buffer
    __shared__ __attribute__((aligned(16))) char s_w[NBUF][kLdsWaves][TB];
    __shared__ qasr::float4v s_acc[NBUF > 1 ? kLdsMaxTiles : 1][kLdsWaves][64];
    __shared__ float s_y[OUT == kOutAcc ? kLdsWaves : 1][256];
    __shared__ __attribute__((aligned(16))) float s_gain[NORM ? kNormMaxK : 1];
    __shared__ float s_part[NORM ? kSkinnyRows * 4 : 1];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int M = p.M, N = p.N, K = p.K;
    const int t0 = blockIdx.x * tpw;
    const int nt = min(tpw, N / 16 - t0);
    const int kbeg = (blockIdx.y * kLdsWaves + wave) * KW;
    constexpr bool kGlu = OUT == kOutGlu;
    // W row of row i (0..15) of column tile t: 16t + i, or for kOutGlu gate
    // rows 8t..8t+7 then up rows N/2 + 8t..
    auto wrow = [&](int t, int i) { return kGlu ? (i < 8 ? 8 * t + i : N / 2 + 8 * t + i - 8) : 16 * t + i; };
    const qasr::u32x4v wres = qasr::make_rsrc_words(p.W, N * K * wbytes);  // < 2^31 (host-checked)
    auto copy_tile = [&](int t, int b) {
#pragma unroll
        for (int i = 0; i < NCP; ++i) {
            const int row = i * RPI + lane / LPR;
            const int chunk = (lane % LPR) ^ row;
            qasr::dma16(wres, wrow(t, row) * K * wbytes + kbeg * wbytes + chunk * 16,
                        qasr::lds_addr(&s_w[b][wave][i * 1024]));
        }
    };

    // The fused norm's loads, the activation slice and (int8) this lane's
    // row scales first, then the first tiles' copies.
    NormPrologue<kLdsWaves> np;
    if constexpr (NORM) np.issue(p, wave, lane);
    const __amdgpu_buffer_rsrc_t xres = rsrc(p.X, (int64_t)M * K * 2);
    qasr::half8v xr[NKS];
#pragma unroll
    for (int s = 0; s < NKS; ++s) xr[s] = load8(xres, (r * K + kbeg + 32 * s + 8 * g) * 2);
    float wsc[kLdsMaxTiles] = {};
    if constexpr (W8) {
#pragma unroll
        for (int t = 0; t < kLdsMaxTiles; ++t)
            if (t < nt) wsc[t] = p.scale[wrow(t0 + t, r)];
    }
    copy_tile(t0, 0);
    if (NBUF > 1 && nt > 1) copy_tile(t0 + 1, 1);
    if constexpr (NORM) {
        const float inv = np.finish(p, s_gain, s_part, wave, lane, r);
#pragma unroll
        for (int s = 0; s < NKS; ++s) {
            const int k = kbeg + 32 * s + 8 * g;
            const float4 g0 = *(const float4*)&s_gain[k];
            const float4 g1 = *(const float4*)&s_gain[k + 4];
            const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) xr[s][e] = f16_of_f32(((float)xr[s][e] * inv) * gv[e]);
        }
    }

    for (int t = 0; t < nt; ++t) {
        const int b = NBUF > 1 ? (t & 1) : 0;
        // This wave's copies of tile t have landed (tile t+1's may not).
        if (NBUF > 1 && t + 1 < nt)
            __builtin_amdgcn_s_waitcnt(0x0F70 | (NCP & 15) | ((NCP >> 4) << 14));  // vmcnt(NCP)
        else
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        const char* buf = &s_w[b][wave][0];
        const float ws = t == 0 ? wsc[0] : t == 1 ? wsc[1] : t == 2 ? wsc[2] : wsc[3];
        qasr::float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < NKS; ++s) {
            const int c = 4 * s + g;  // this k-step's 8 weights: bytes [c * 8 wbytes, +8 wbytes)
            qasr::half8v bw;
            if constexpr (W8) {
                const uint2 q = *(const uint2*)(buf + r * RB + (((c >> 1) ^ r) * 16) + (c & 1) * 8);
                bw = dequant8(q.x, q.y, ws);
            } else {
                bw = *(const qasr::half8v*)(buf + r * RB + ((c ^ r) * 16));
            }
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xr[s], bw, acc, 0, 0, 0);
        }
        s_acc[t][wave][lane] = acc;
        if (t + NBUF < nt) {
            // Refill this buffer once this wave's reads of it have returned.
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            copy_tile(t0 + t + NBUF, b);
        }
    }
    __syncthreads();
    for (int t = wave; t < nt; t += kLdsWaves) {
        qasr::float4v sum = s_acc[t][0][lane];
#pragma unroll
        for (int w = 1; w < kLdsWaves; ++w) sum += s_acc[t][w][lane];
        skinny_tile_out<OUT>(p, sum, t0 + t, blockIdx.y, lane, s_y[OUT == kOutAcc ? wave : 0]);
    }
}

// ---- skinny GEMM with the activation rows shared in LDS ---------------------
// The product of skinny_gemm_kernel, with its K slices and summation order,
// for wide outputs: a workgroup takes TPW consecutive column tiles with KS
// waves each (wave w: tile w / KS, K slice w % KS of the workgroup's K
// range), and the 16 activation rows of that K range are read once into LDS
// -- normed there once when NORM, as skinny_gemm_kernel norms them on their
// way into the MFMA -- and shared by the TPW tiles.  skinny_gemm_kernel
// requests them again for every tile: at 16 rows as many bytes, from L2, as
// the weights it streams.  The weights still go straight from the buffer
// loads into the MFMA B operand, two stages of U k-steps in flight per wave.
// Activation rows are padded by 16 bytes, so the 16-row operand read hits 16
// different bank groups.  The results equal skinny_gemm_kernel's bit for bit.
constexpr int kSharedMaxK = 3072;  // K per workgroup (the K range of one group)
constexpr int kSharedPad = 8;      // halves of padding per activation row

template <int KS, int TPW, int KMAX, bool W8, int OUT, bool NORM>
__global__ __launch_bounds__(KS * TPW * 64) void skinny_shared_kernel(SkinnyArgs p) {
    constexpr int NW = KS * TPW, NT = NW * 64;
    constexpr int U = kSkinnyUnroll;
    constexpr int AROW = KMAX + kSharedPad;
    static_assert(kSkinnyRows * AROW * 2 >= NW * 64 * 16, "the partials reuse the activation rows");
    __shared__ __attribute__((aligned(16))) f16 s_act[kSkinnyRows * AROW];
    // After the MFMAs the activation rows hold the per-wave partials.
    qasr::float4v(*s_red)[64] = reinterpret_cast<qasr::float4v(*)[64]>(s_act);
    __shared__ __attribute__((aligned(16))) float s_gain[NORM ? kNormMaxK : 1];
    __shared__ float s_part[NORM ? kSkinnyRows * 4 : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int M = p.M, N = p.N, K = p.K, groups = p.groups;
    const int t = wave / KS, ks = wave % KS;
    const int ntiles = N / 16;
    const int tile = blockIdx.x * TPW + t;
    const bool tile_ok = tile < ntiles;
    const int tile_c = tile_ok ? tile : ntiles - 1;  // a wave past the last tile streams a real one, unused
    const int kg = K / groups, kbase = blockIdx.y * kg;
    const int kw = kg / KS, kbeg = kbase + ks * kw;
    constexpr int wbytes = W8 ? 1 : 2;
    constexpr bool kGlu = OUT == kOutGlu;
    const int n0 = tile_c * 16;
    const int w0 = kGlu ? 8 * tile_c : n0;
    const int rr = kGlu ? (r < 8 ? r : N / 2 + r - 8) : r;
    const int64_t wrows = kGlu ? (int64_t)(N / 2 + 8) : 16;
    const __amdgpu_buffer_rsrc_t wres =
        rsrc((const char*)p.W + (int64_t)w0 * K * wbytes, wrows * K * wbytes);
    float wsc = 0.0f;
    if constexpr (W8) wsc = p.scale[w0 + rr];
    const int woff = rr * K * 2 + g * 16;

    struct Stage {
        qasr::half8v b[U];
        uint2 q[U];
    };
    const int nst = kw / (32 * U);
    auto load_stage = [&](int st, Stage& S) {
        const int k0 = kbeg + st * 32 * U;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kk = k0 + 32 * u;
            if constexpr (W8)
                S.q[u] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wres, rr * K + g * 8 + kk, 0, 0));
            else
                S.b[u] = load8(wres, woff + kk * 2);
        }
    };
    // The residual of this tile's outputs (kOutAcc), ahead of the stream.
    f16 y_pre[4] = {};
    if constexpr (OUT == kOutAcc) {
        if (ks == 0 && tile_ok) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (4 * g + i < M) y_pre[i] = ((const f16*)p.Y)[(int64_t)(4 * g + i) * N + n0 + r];
        }
    }
    NormPrologue<NW> np;
    if constexpr (NORM) np.issue(p, wave, lane);
    // The workgroup's activation rows: piece q = threadIdx.x + i NT is row
    // q % 16 (= r, this lane's row: NT is a multiple of 16), chunk q / 16 of 8
    // values; rows past M read as zeros.  Up to 8 pieces per thread and round.
    // The first round is requested before the weight stages and the second
    // stage after the rows are staged: requests return in order, so rows
    // requested behind both stages would wait for them.
    const int nchunk = kg / 8, npieces = kSkinnyRows * nchunk;
    auto load_pieces = [&](int base, uint4 (&x)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = base + threadIdx.x + i * NT, c = q >> 4;
            x[i] = (q < npieces && r < M) ? *(const uint4*)(p.X + (int64_t)r * K + kbase + 8 * c)
                                          : make_uint4(0, 0, 0, 0);
        }
    };
    uint4 x0[8];
    load_pieces(0, x0);
    Stage s0, s1;
    load_stage(0, s0);
    float inv = 0.0f;
    if constexpr (NORM) inv = np.finish(p, s_gain, s_part, wave, lane, r);
    for (int base = 0; base < npieces; base += 8 * NT) {
        uint4 x[8];
        if (base == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = x0[i];
        } else {
            load_pieces(base, x);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = base + threadIdx.x + i * NT, c = q >> 4;
            if (q >= npieces) continue;
            H8 v;
            v.u = x[i];
            if constexpr (NORM) {
                const float* gv = &s_gain[kbase + 8 * c];
#pragma unroll
                for (int e = 0; e < 8; ++e) v.e[e] = f16_of_f32(((float)v.e[e] * inv) * gv[e]);
            }
            *(uint4*)&s_act[r * AROW + 8 * c] = v.u;
        }
    }
    load_stage(1, s1);
    __syncthreads();

    qasr::float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const f16* arow = &s_act[r * AROW + 8 * g];
    auto mma_stage = [&](const Stage& S, int st) {
        const int k0 = kbeg - kbase + st * 32 * U;  // within the workgroup's K range
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const qasr::half8v xa = *(const qasr::half8v*)&arow[k0 + 32 * u];
            if constexpr (W8) {
                const qasr::half8v b = dequant8(S.q[u].x, S.q[u].y, wsc);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, b, acc, 0, 0, 0);
            } else {
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, S.b[u], acc, 0, 0, 0);
            }
        }
    };
    int st = 0;
    for (; st + 2 < nst; st += 2) {
        __builtin_amdgcn_sched_barrier(0);
        mma_stage(s0, st);
        __builtin_amdgcn_sched_barrier(0);
        load_stage(st + 2, s0);
        __builtin_amdgcn_sched_barrier(0);
        mma_stage(s1, st + 1);
        __builtin_amdgcn_sched_barrier(0);
        load_stage(st + 3, s1);
    }
    __builtin_amdgcn_sched_barrier(0);
    mma_stage(s0, st);
    __builtin_amdgcn_sched_barrier(0);
    mma_stage(s1, st + 1);
    __syncthreads();  // every wave is done reading the activation rows
    s_red[wave][lane] = acc;
    __syncthreads();
    if (ks != 0 || !tile_ok) return;
    qasr::float4v sum = s_red[t * KS][lane];
#pragma unroll
    for (int w = 1; w < KS; ++w) sum += s_red[t * KS + w][lane];
    skinny_tile_out<OUT>(p, sum, tile, blockIdx.y, lane, reinterpret_cast<float*>(&s_red[t * KS][0]),
                         OUT == kOutAcc ? y_pre : nullptr);
}

// ---- skinny GEMM with several column tiles per wave ------------------------
// The product of skinny_gemm_kernel, each wave taking TW consecutive column
// tiles over its K slice: one activation load per k-step feeds TW MFMAs
// (skinny_gemm_kernel loads the activations again for every tile).  A
// workgroup of KS waves covers TW tiles with K cut KS ways, the K slices and
// summation order of skinny_gemm_kernel's KS waves, so the results are
// bitwise its results.  For the 1.7B gate|up (f16) four tiles per wave took
// the 16-slot step from 1917 us (skinny_shared_kernel) to 1898 us; two
// tiles, or the narrower projections (fewer workgroups than CUs), measured
// slower, and so did int8 weights, whose dequantisation then runs on one
// wave per SIMD (1904 against 1837 us).
template <int KS, int TW, int U, bool W8, int OUT, bool NORM>
__global__ __launch_bounds__(KS * 64) void skinny_multi_kernel(SkinnyArgs p) {
    static_assert(TW <= KS, "one epilogue wave per tile");
    __shared__ qasr::float4v s_red[TW][KS][64];
    __shared__ __attribute__((aligned(16))) float s_gain[NORM ? kNormMaxK : 1];
    __shared__ float s_part[NORM ? kSkinnyRows * 4 : 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int M = p.M, N = p.N, K = p.K, groups = p.groups;
    const int ntiles = N / 16;
    const int t0 = blockIdx.x * TW;
    const int kw = K / (KS * groups);
    const int kbeg = (blockIdx.y * KS + wave) * kw;
    constexpr int wbytes = W8 ? 1 : 2;
    constexpr bool kGlu = OUT == kOutGlu;
    // Weight row of this lane in tile j (clamped to the last tile: a tile
    // past the end streams a real one, unused).
    __amdgpu_buffer_rsrc_t wres[TW];
    float wsc[TW];
    int rrow[TW];
#pragma unroll
    for (int j = 0; j < TW; ++j) {
        const int tile = min(t0 + j, ntiles - 1);
        const int w0 = kGlu ? 8 * tile : tile * 16;
        rrow[j] = kGlu ? (r < 8 ? r : N / 2 + r - 8) : r;
        const int64_t wrows = kGlu ? (int64_t)(N / 2 + 8) : 16;
        wres[j] = rsrc((const char*)p.W + (int64_t)w0 * K * wbytes, wrows * K * wbytes);
        wsc[j] = 0.0f;
        if constexpr (W8) wsc[j] = p.scale[w0 + rrow[j]];
    }
    const __amdgpu_buffer_rsrc_t xres = rsrc(p.X, (int64_t)M * K * 2);
    const int xoff = r * K * 2 + g * 16;
    struct Stage {
        qasr::half8v b[TW][U], x[U];
        uint2 q[TW][U];
    };
    const int nst = kw / (32 * U);
    auto load_stage = [&](int st, Stage& S) {
        const int k0 = kbeg + st * 32 * U;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kk = k0 + 32 * u;
#pragma unroll
            for (int j = 0; j < TW; ++j) {
                if constexpr (W8)
                    S.q[j][u] = __builtin_bit_cast(
                        uint2, __builtin_amdgcn_raw_buffer_load_b64(wres[j], rrow[j] * K + g * 8 + kk, 0, 0));
                else
                    S.b[j][u] = load8(wres[j], rrow[j] * K * 2 + g * 16 + kk * 2);
            }
            S.x[u] = load8(xres, xoff + kk * 2);
        }
    };
    qasr::float4v acc[TW];
#pragma unroll
    for (int j = 0; j < TW; ++j) acc[j] = qasr::float4v{0.0f, 0.0f, 0.0f, 0.0f};
    float inv = 0.0f;
    auto act = [&](const qasr::half8v& x, int kk) {
        if constexpr (NORM) {
            const float4 g0 = *(const float4*)&s_gain[kk + 8 * g];
            const float4 g1 = *(const float4*)&s_gain[kk + 8 * g + 4];
            const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
            qasr::half8v n;
#pragma unroll
            for (int e = 0; e < 8; ++e) n[e] = f16_of_f32(((float)x[e] * inv) * gv[e]);
            return n;
        } else {
            return x;
        }
    };
    auto mma_stage = [&](const Stage& S, int st) {
        const int k0 = kbeg + st * 32 * U;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const qasr::half8v xa = act(S.x[u], k0 + 32 * u);
#pragma unroll
            for (int j = 0; j < TW; ++j) {
                if constexpr (W8) {
                    const qasr::half8v b = dequant8(S.q[j][u].x, S.q[j][u].y, wsc[j]);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, b, acc[j], 0, 0, 0);
                } else {
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, S.b[j][u], acc[j], 0, 0, 0);
                }
            }
        }
    };
    // The residual of the tile this wave finishes (kOutAcc), ahead of the stream.
    f16 y_pre[4] = {};
    const int my_tile = t0 + wave;  // the tile this wave finishes, if wave < TW
    if constexpr (OUT == kOutAcc) {
        if (wave < TW && my_tile < ntiles) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (4 * g + i < M) y_pre[i] = ((const f16*)p.Y)[(int64_t)(4 * g + i) * N + my_tile * 16 + r];
        }
    }
    Stage s0, s1;
    NormPrologue<KS> np;
    if constexpr (NORM) np.issue(p, wave, lane);
    // The second stage is requested after the folded norm's inputs have
    // arrived: requested together, they queued behind the weight stages.
    load_stage(0, s0);
    if constexpr (NORM) inv = np.finish(p, s_gain, s_part, wave, lane, r);
    load_stage(1, s1);
    int st = 0;
    for (; st + 2 < nst; st += 2) {
        __builtin_amdgcn_sched_barrier(0);
        mma_stage(s0, st);
        __builtin_amdgcn_sched_barrier(0);
        load_stage(st + 2, s0);
        __builtin_amdgcn_sched_barrier(0);
        mma_stage(s1, st + 1);
        __builtin_amdgcn_sched_barrier(0);
        load_stage(st + 3, s1);
    }
    __builtin_amdgcn_sched_barrier(0);
    mma_stage(s0, st);
    __builtin_amdgcn_sched_barrier(0);
    mma_stage(s1, st + 1);
#pragma unroll
    for (int j = 0; j < TW; ++j) s_red[j][wave][lane] = acc[j];
    __syncthreads();
    if (wave >= TW || my_tile >= ntiles) return;
    qasr::float4v sum = s_red[wave][0][lane];
#pragma unroll
    for (int w = 1; w < KS; ++w) sum += s_red[wave][w][lane];
    skinny_tile_out<OUT>(p, sum, my_tile, blockIdx.y, lane, reinterpret_cast<float*>(&s_red[wave][0][0]),
                         OUT == kOutAcc ? y_pre : nullptr);
}

const char* blas_msg(rocblas_status st) { return rocblas_status_to_string(st); }

}  // namespace

struct qasr_decoder {
    qasr_ctx* ctx = nullptr;
    qasr_decoder_cfg cfg{};
    const f16* embed = nullptr;
    const f16* final_norm = nullptr;
    std::vector<qasr_layer_weights> layers;
    rocblas_handle blas = nullptr;
    void* blas_ws = nullptr;
    hipStream_t stream = nullptr;  // of the call in progress
    bool force_blas = false;       // QASR_DECODER_BLAS=1: every projection through rocBLAS
    bool fuse = true;              // QASR_DECODER_FUSE=0: no fused epilogues (same results)
    int lds_gemm = 1;              // QASR_SKINNY_LDS: 0 older kernel only, 2 LDS kernel wherever it fits
    int lds_tpw = 0, lds_groups = 0;  // QASR_SKINNY_TPW / _GROUPS: shape overrides (0 = planner)
    bool own_gemm = true;             // QASR_PREFILL_GEMM=blas: rocBLAS for the prefill projections instead
    bool prefill = false;             // inside a prefill's layers: every projection takes the GEMM
    int shared_tiles = 3;             // QASR_SKINNY_SHARED: skinny_shared_kernel tiles per workgroup (0 off)
    int shared_min_tiles = 512;       // QASR_SKINNY_SHARED_MIN_TILES: narrower outputs keep skinny_gemm_kernel
    bool argmax_tiles = true;         // QASR_ARGMAX_TILES=0: the two-pass argmax over the logits
    int multi_tiles = -1;             // QASR_SKINNY_MULTI: skinny_multi_kernel tiles per wave (0 off, -1 by width)
    // activations, max_rows rows each
    f16* x = nullptr;     // residual stream [rows][hs]
    f16* n = nullptr;     // normed rows [rows][hs]
    f16* qkv = nullptr;   // [rows][(nqh + 2 nkvh) hd]
    f16* qw = nullptr;    // roped q of a prefill [rows][nqh hd]
    f16* attn = nullptr;  // [rows][nqh hd]
    f16* gu = nullptr;    // [rows][2 inter]
    f16* h = nullptr;     // [rows][inter]
    float* logits = nullptr;  // [kHeadRows][vocab]
    float* am_v = nullptr;    // argmax candidates [kHeadRows][kArgmaxChunks] or [kSkinnyRows][vocab / 16]
    int* am_i = nullptr;
    // split projections: partials [tile][group][64 lanes][4] and one arrival
    // ticket per column tile (zero at rest: the last arrival resets it)
    float* sk_ws = nullptr;
    uint32_t* sk_ctr = nullptr;
    f16* wdq = nullptr;      // int8 projections of prefill calls: one dequantised matrix
    int64_t wdq_elems = 0;
    // Chunk sums of squares of the residual rows [kSkinnyRows][kNormMaxChunks],
    // written by the launch that last wrote x when ss_valid (embedding or a
    // skinny residual projection): a fused RMSNorm's starting point.
    float* ss = nullptr;
    bool ss_valid = false;
};

namespace {

void free_decoder(qasr_decoder* d) {
    if (d->blas) (void)rocblas_destroy_handle(d->blas);
    for (void* p : {(void*)d->blas_ws, (void*)d->x, (void*)d->n, (void*)d->qkv, (void*)d->qw,
                    (void*)d->attn, (void*)d->gu, (void*)d->h, (void*)d->logits, (void*)d->am_v,
                    (void*)d->am_i, (void*)d->sk_ws, (void*)d->sk_ctr, (void*)d->wdq, (void*)d->ss})
        if (p) (void)hipFree(p);
    delete d;
}

// y[rows][n_out] = f16(x[rows][k] . W[n_out][k]^T (+ y)), f32 accumulation.
// Row-major [rows][k] is column-major k x rows, so y^T = W . x^T is
// op(A) = W^T of the column-major k x n_out array W.
// Launch shape of an n_out x k projection (measured on MI355X at the 0.6B and
// 1.7B shapes): column tiles that fill the GPU (>= kSkinnyTargetWgs) take 4
// waves; fewer tiles take the most of {12, 8, 4} waves whose K slices are
// whole stage pairs, and a long K (>= 4096) is also cut into `groups` ranges
// across workgroups until the launch has kSkinnySplitWgs workgroups (the
// partial merge costs ~2 us, repaid only by a long stream; at 2048 x 6144,
// 2 groups beat 1, 3 and 6 by 20-65 us per 28-layer step, f16 and int8
// alike).  ks = 0: not a skinny shape (rocBLAS then).
// The LDS-staged kernel (nks > 0) takes very wide outputs (at least
// kLdsMinTiles column tiles: the logits' 9,496) of at least kLdsMinRows
// activation rows whose K splits into 4 waves x `groups` slices of 512 or 256
// weights, 4 column tiles per workgroup: there one activation slice in
// registers serves four tiles, and the lm_head step measured 135 us against
// 161 us (1.7B, 16 rows; the whole step 1.976 against 2.003 ms).  With one
// row there are no activation bytes to save and it lost (0.6B step 0.989
// against 0.974 ms).  At the projections' widths
// (128-768 tiles) it measured no faster than skinny_gemm_kernel (qkv 8.7
// against 8.4 us, gate|up 18.4 against 17.5 us), so those keep it.
// QASR_SKINNY_LDS=0 / =2 select the older kernel everywhere / the LDS kernel
// at every shape it takes; QASR_SKINNY_TPW / QASR_SKINNY_GROUPS override its
// tiles per workgroup and K groups (sweeps).
struct SkinnyShape {
    int ks = 0, groups = 1;
    int nks = 0, tpw = 1, nbuf = 1;  // nks > 0: skinny_lds_kernel
    int shared_tiles = 0;            // > 1: skinny_shared_kernel, this many tiles per workgroup
    int multi_tiles = 0, multi_ks = 0;  // > 1: skinny_multi_kernel, tiles per wave and waves
};

SkinnyShape lds_shape(qasr_decoder* d, int rows, int n_out, int k, bool w8) {
    SkinnyShape sh{};
    const int tiles = n_out / 16;
    if ((int64_t)n_out * k * (w8 ? 1 : 2) >= (int64_t(1) << 31)) return sh;
    if ((tiles < kLdsMinTiles || rows < kLdsMinRows) && d->lds_gemm < 2) return sh;
    for (int g = 1; g <= kSkinnyMaxGroups && !sh.nks; ++g) {
        if (d->lds_groups > 0 && g != d->lds_groups) continue;
        if (k % (4 * g)) continue;
        const int kw = k / (4 * g);
        if ((kw == 512 || kw == 256) && (g == 1 || tiles <= kSkinnyMaxTiles)) {
            sh.nks = kw / 32;
            sh.groups = g;
        }
    }
    if (!sh.nks) return sh;
    sh.tpw = d->lds_tpw > 0 ? std::min(d->lds_tpw, kLdsMaxTiles) : (tiles >= kLdsMinTiles ? 4 : 1);
    if (sh.groups > 1) sh.tpw = 1;
    sh.nbuf = sh.tpw > 1 ? 2 : 1;  // tpw == 1 <=> one buffer (s_acc holds one tile then)
    return sh;
}

SkinnyShape skinny_base_shape(qasr_decoder* d, int rows, int n_out, int k, bool w8, bool allow_lds) {
    if (d->force_blas || d->prefill || rows > kSkinnyRows || n_out % 16) return SkinnyShape{};
    if (d->lds_gemm && allow_lds) {
        const SkinnyShape sh = lds_shape(d, rows, n_out, k, w8);
        if (sh.nks) return sh;
    }
    const int tiles = n_out / 16;
    if (tiles >= kSkinnyTargetWgs) return SkinnyShape{k % (4 * kSkinnyPair) ? 0 : 4, 1};
    // K of 3072 or more is cut across workgroups (the down_proj of both shapes):
    // two groups reach 256 workgroups at the 1.7B shape; the 0.6B's 64 tiles
    // take three (192; one-slot step 956 against 962 us unsplit).  K = 2048
    // stays whole (16-slot step 1810 against 1847 us split).
    if (k >= kSkinnySplitMinK) {
        int best = 0;
        for (int g : {2, 3, 4, 6, 8, 12})
            if (k % (4 * g * kSkinnyPair) == 0) {
                best = g;
                if (tiles * g >= kSkinnySplitWgs) break;
            }
        if (best) return SkinnyShape{4, best};
    }
    for (int ks : {12, 8, 4})
        if (k % (ks * kSkinnyPair) == 0) return SkinnyShape{ks, 1};
    return SkinnyShape{};
}

// Tiles per workgroup of skinny_shared_kernel for a base shape, or 0 where
// it does not apply: fewer than kSharedMinRows rows, or outputs narrower than
// QASR_SKINNY_SHARED_MIN_TILES column tiles (512: 1.7B gate|up).  Three tiles
// of four waves took the 1.7B 16-slot gate|up from 17.1 to 16.1 us and the
// whole step from 1929 to 1913 us (int8: 1902 to 1835 us, where the per-tile
// kernel's activation bytes are twice its weight bytes); four tiles, or
// narrower projections (down_proj 11.8 -> 17.0 us at three tiles: too few
// workgroups) measured slower.
// QASR_SKINNY_SHARED: 0 never, T forces T tiles.
int shared_tiles(qasr_decoder* d, const SkinnyShape& sh, int rows, int n_out, int k) {
    if (!sh.ks || sh.nks || rows < kSharedMinRows || k / sh.groups > kSharedMaxK) return 0;
    const int want = d->shared_tiles;
    if (want == 0) return 0;
    const int tiles = n_out / 16;
    if (tiles < d->shared_min_tiles) return 0;
    for (int t : {4, 3, 2}) {
        if (want > 1 && t != want) continue;
        if (sh.ks * t <= 16 && (sh.ks == 4 || t == 2) && tiles >= t) return t;
    }
    return 0;
}

SkinnyShape skinny_shape(qasr_decoder* d, int rows, int n_out, int k, bool w8 = false) {
    // Wide outputs of at least kSharedMinRows rows: f16 weights take several
    // tiles per wave (skinny_multi_kernel; the logits too, 1889 against 1897
    // us per 16-slot step with skinny_lds_kernel), int8 weights the LDS-shared
    // activation rows (skinny_shared_kernel), whose twelve waves hide the
    // dequantisation better.  Both keep the base shape's K slices.  Tiles per
    // wave: the fewest (two to four) that need no more than one workgroup per
    // CU -- the 1.7B gate|up's 768 tiles take three (256 workgroups: 14.1 us
    // against 15.6 with four on 192), the logits' 9,496 four (126.9 against
    // 130.5 us with three).  QASR_SKINNY_MULTI=T forces T (0: off).
    // The choice is made for kSkinnyRows rows whatever the batch's row count
    // (up to kSkinnyRows): the kernels' K slicing, and so every row's bits,
    // must not depend on how many other rows share the launch (the
    // reference's --batch N == --batch 1, decoder.rs:686-693).
    if (rows > kSkinnyRows) return SkinnyShape{};
    const int sr = kSkinnyRows;
    const int tiles = n_out / 16, cus = std::max(d->ctx->cus, 1);
    const int tw = d->multi_tiles < 0 ? std::min(4, std::max(2, (tiles + cus - 1) / cus)) : d->multi_tiles;
    const bool multi_ok = !w8 && tw > 1 && sr >= kSharedMinRows && n_out / 16 >= d->shared_min_tiles &&
                          d->lds_gemm < 2;
    SkinnyShape sh = skinny_base_shape(d, sr, n_out, k, w8, !multi_ok);
    const bool wide = sh.ks && !sh.nks && sr >= kSharedMinRows && n_out / 16 >= d->shared_min_tiles;
    if (wide && !w8 && tw > 1 && (sh.ks == 4 || sh.ks == 8) && (tw >= 2 && tw <= 4)) {
        sh.multi_tiles = tw;
        sh.multi_ks = sh.ks;
        return sh;
    }
    sh.shared_tiles = shared_tiles(d, sh, sr, n_out, k);
    return sh;
}

template <bool W8, int OUT, bool NORM>
int launch_skinny_w(qasr_decoder* d, SkinnyShape sh, const SkinnyArgs& a) {
    const dim3 grid(a.N / 16, sh.groups);
    constexpr int U = kSkinnyUnroll;
    switch (sh.ks) {
        case 4:
            hipLaunchKernelGGL((skinny_gemm_kernel<4, U, W8, OUT, NORM>), grid, dim3(4 * 64), 0,
                               d->stream, a);
            break;
        case 8:
            hipLaunchKernelGGL((skinny_gemm_kernel<8, U, W8, OUT, NORM>), grid, dim3(8 * 64), 0,
                               d->stream, a);
            break;
        case 12:
            hipLaunchKernelGGL((skinny_gemm_kernel<12, U, W8, OUT, NORM>), grid, dim3(12 * 64),
                               0, d->stream, a);
            break;
        default:
            return fail(QASR_EINVAL, "skinny GEMM: %d waves", sh.ks);
    }
    HIP_TRY(hipGetLastError(), "projection launch");
    return QASR_OK;
}

template <bool W8, int OUT, bool NORM>
int launch_skinny_lds(qasr_decoder* d, SkinnyShape sh, const SkinnyArgs& a) {
    const dim3 grid((a.N / 16 + sh.tpw - 1) / sh.tpw, sh.groups);
    const dim3 block(kLdsWaves * 64);
    if (sh.nks == 16 && sh.nbuf == 2)
        hipLaunchKernelGGL((skinny_lds_kernel<16, W8, OUT, NORM, 2>), grid, block, 0, d->stream, a, sh.tpw);
    else if (sh.nks == 16)
        hipLaunchKernelGGL((skinny_lds_kernel<16, W8, OUT, NORM, 1>), grid, block, 0, d->stream, a, sh.tpw);
    else if (sh.nks == 8 && sh.nbuf == 2)
        hipLaunchKernelGGL((skinny_lds_kernel<8, W8, OUT, NORM, 2>), grid, block, 0, d->stream, a, sh.tpw);
    else if (sh.nks == 8)
        hipLaunchKernelGGL((skinny_lds_kernel<8, W8, OUT, NORM, 1>), grid, block, 0, d->stream, a, sh.tpw);
    else
        return fail(QASR_EINVAL, "skinny GEMM: %d k-steps per wave", sh.nks);
    HIP_TRY(hipGetLastError(), "projection launch");
    return QASR_OK;
}

template <bool W8, int OUT, bool NORM>
int launch_skinny_shared(qasr_decoder* d, SkinnyShape sh, const SkinnyArgs& a) {
    const int t = sh.shared_tiles;
    const dim3 grid((a.N / 16 + t - 1) / t, sh.groups);
    const bool k2 = a.K / sh.groups <= 2048;  // 66 KB of activation rows: two workgroups per CU
    if (sh.ks == 4 && t == 4 && k2)
        hipLaunchKernelGGL((skinny_shared_kernel<4, 4, 2048, W8, OUT, NORM>), grid, dim3(16 * 64), 0, d->stream, a);
    else if (sh.ks == 4 && t == 4)
        hipLaunchKernelGGL((skinny_shared_kernel<4, 4, kSharedMaxK, W8, OUT, NORM>), grid, dim3(16 * 64), 0, d->stream, a);
    else if (sh.ks == 4 && t == 3 && k2)
        hipLaunchKernelGGL((skinny_shared_kernel<4, 3, 2048, W8, OUT, NORM>), grid, dim3(12 * 64), 0, d->stream, a);
    else if (sh.ks == 4 && t == 3)
        hipLaunchKernelGGL((skinny_shared_kernel<4, 3, kSharedMaxK, W8, OUT, NORM>), grid, dim3(12 * 64), 0, d->stream, a);
    else if (sh.ks == 4 && t == 2 && k2)
        hipLaunchKernelGGL((skinny_shared_kernel<4, 2, 2048, W8, OUT, NORM>), grid, dim3(8 * 64), 0, d->stream, a);
    else if (sh.ks == 4 && t == 2)
        hipLaunchKernelGGL((skinny_shared_kernel<4, 2, kSharedMaxK, W8, OUT, NORM>), grid, dim3(8 * 64), 0, d->stream, a);
    else if (sh.ks == 8 && t == 2 && k2)
        hipLaunchKernelGGL((skinny_shared_kernel<8, 2, 2048, W8, OUT, NORM>), grid, dim3(16 * 64), 0, d->stream, a);
    else if (sh.ks == 8 && t == 2)
        hipLaunchKernelGGL((skinny_shared_kernel<8, 2, kSharedMaxK, W8, OUT, NORM>), grid, dim3(16 * 64), 0, d->stream, a);
    else
        return fail(QASR_EINVAL, "skinny GEMM: %d waves x %d shared tiles", sh.ks, t);
    HIP_TRY(hipGetLastError(), "projection launch");
    return QASR_OK;
}

template <bool W8, int OUT, bool NORM>
int launch_skinny_multi(qasr_decoder* d, SkinnyShape sh, const SkinnyArgs& a) {
    const int tw = sh.multi_tiles, ks = sh.multi_ks;
    const dim3 grid((a.N / 16 + tw - 1) / tw, sh.groups);
    constexpr int U = kSkinnyUnroll;
#define QASR_MULTI(KS_, TW_)                                                                      \
    else if (ks == KS_ && tw == TW_) hipLaunchKernelGGL((skinny_multi_kernel<KS_, TW_, U, W8, OUT, NORM>), \
                                                        grid, dim3(KS_ * 64), 0, d->stream, a);
    if (false) {
    }
    QASR_MULTI(4, 2) QASR_MULTI(8, 2) QASR_MULTI(4, 3) QASR_MULTI(8, 3) QASR_MULTI(4, 4) QASR_MULTI(8, 4)
    else return fail(QASR_EINVAL, "skinny GEMM: %d waves x %d tiles per wave", ks, tw);
#undef QASR_MULTI
    HIP_TRY(hipGetLastError(), "projection launch");
    return QASR_OK;
}

template <int OUT, bool NORM = false>
int launch_skinny(qasr_decoder* d, SkinnyShape sh, const SkinnyArgs& a) {
    if (sh.multi_tiles > 1)
        return a.scale ? launch_skinny_multi<true, OUT, NORM>(d, sh, a)
                       : launch_skinny_multi<false, OUT, NORM>(d, sh, a);
    if (sh.shared_tiles > 1)
        return a.scale ? launch_skinny_shared<true, OUT, NORM>(d, sh, a)
                       : launch_skinny_shared<false, OUT, NORM>(d, sh, a);
    if (sh.nks)
        return a.scale ? launch_skinny_lds<true, OUT, NORM>(d, sh, a)
                       : launch_skinny_lds<false, OUT, NORM>(d, sh, a);
    return a.scale ? launch_skinny_w<true, OUT, NORM>(d, sh, a)
                   : launch_skinny_w<false, OUT, NORM>(d, sh, a);
}

SkinnyArgs skinny_args(qasr_decoder* d, SkinnyShape sh, int rows, int n_out, int k, const void* W,
                       const f16* x, void* y, const float* scale = nullptr) {
    SkinnyArgs a{};
    a.W = W;
    a.scale = scale;
    a.X = x;
    a.Y = y;
    a.M = rows;
    a.N = n_out;
    a.K = k;
    a.groups = sh.groups;
    a.ws = d->sk_ws;
    a.counters = d->sk_ctr;
    return a;
}

// y = x . W^T (+ y).  W is f16, or int8 with per-row `scale`.  Skinny shapes
// run the MFMA skinny kernel (int8 dequantised in registers); others go to
// rocBLAS, an int8 W first dequantised into the scratch matrix.
int gemm_f16(qasr_decoder* d, int rows, int n_out, int k, const void* W, const f16* x, f16* y,
             bool accumulate, const float* scale = nullptr) {
    const SkinnyShape sh = skinny_shape(d, rows, n_out, k, scale != nullptr);
    if (y == d->x) d->ss_valid = false;  // unless the launch below writes the chunk sums
    if (sh.ks || sh.nks) {
        SkinnyArgs a = skinny_args(d, sh, rows, n_out, k, W, x, y, scale);
        if (accumulate && y == d->x && d->fuse && n_out <= kNormMaxK) {
            a.ss_out = d->ss;  // the residual rows' chunk sums, for the next fused norm
            d->ss_valid = true;
        }
        return accumulate ? launch_skinny<kOutAcc>(d, sh, a) : launch_skinny<kOutF16>(d, sh, a);
    }
    if (scale) {
        if (!d->wdq || (int64_t)n_out * k > d->wdq_elems)
            return fail(QASR_EINVAL, "int8 projection %dx%d without dequantisation scratch", n_out, k);
        const int64_t groups8 = (int64_t)n_out * k / 8;
        hipLaunchKernelGGL(dequant_rows_kernel, dim3((unsigned)((groups8 + 255) / 256)), dim3(256),
                           0, d->stream, (const int8_t*)W, scale, (int64_t)n_out, k, d->wdq);
        HIP_TRY(hipGetLastError(), "dequantisation launch");
        W = d->wdq;
    }
    if (d->own_gemm && qasr::gemm_f16_fits(rows, n_out, k)) {
        HIP_TRY(qasr::launch_gemm_f16(x, (const f16*)W, y, rows, n_out, k, accumulate, d->ctx->cus,
                                      d->stream),
                "projection GEMM launch");
        return QASR_OK;
    }
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    const rocblas_status st = rocblas_gemm_ex(
        d->blas, rocblas_operation_transpose, rocblas_operation_none, n_out, rows, k, &alpha, W,
        rocblas_datatype_f16_r, k, x, rocblas_datatype_f16_r, k, &beta, y, rocblas_datatype_f16_r,
        n_out, y, rocblas_datatype_f16_r, n_out, rocblas_datatype_f32_r,
        rocblas_gemm_algo_standard, 0, 0);
    if (st != rocblas_status_success) return fail(QASR_EDEVICE, "rocblas_gemm_ex: %s", blas_msg(st));
    return QASR_OK;
}

int launch_rms_norm(const f16* x, int64_t x_stride, const void* w, f16* out, int rows, int hs,
                    float eps, hipStream_t st);

// Whether a projection of the residual rows x (k = hidden size) can take
// its RMSNorm in the skinny kernel's prologue: a skinny shape, and chunk sums
// of x written by the launch that wrote x.
bool norm_fusable(qasr_decoder* d, SkinnyShape sh, int k, const f16* x) {
    return d->fuse && (sh.ks || sh.nks) && k <= kNormMaxK && x == d->x && d->ss_valid;
}

SkinnyArgs with_norm(qasr_decoder* d, SkinnyArgs a, const void* nw) {
    a.nw = (const f16*)nw;
    a.eps = d->ctx->cfg.rms_norm_eps;
    a.ss_in = d->ss;
    return a;
}

// h[rows][inter] = SiLU(x . Wg^T) * (x . Wu^T) for the fused gate|up W in
// one skinny launch (kOutGlu), with x first normed by gain nw when nw is
// set; *fused = false (nothing launched) when the shape or the options rule
// that out.
int glu_skinny(qasr_decoder* d, int rows, int inter, int k, const void* W, const f16* x, f16* h,
               const float* scale, const void* nw, bool* fused) {
    *fused = false;
    if (!d->fuse) return QASR_OK;
    const SkinnyShape sh = skinny_shape(d, rows, 2 * inter, k, scale != nullptr);
    const int64_t span = (int64_t)(inter + 8) * k * (scale ? 1 : 2);
    if (!(sh.ks || sh.nks) || span >= (int64_t(1) << 31)) return QASR_OK;
    if (nw && !norm_fusable(d, sh, k, x)) return QASR_OK;
    *fused = true;
    const SkinnyArgs a = skinny_args(d, sh, rows, 2 * inter, k, W, x, h, scale);
    return nw ? launch_skinny<kOutGlu, true>(d, sh, with_norm(d, a, nw))
              : launch_skinny<kOutGlu>(d, sh, a);
}

// y = f16(rms_norm(x; nw) . W^T): in one skinny launch when the shape
// allows, else rms_norm_kernel into the normed-rows buffer and the
// projection (bit-identical either way).
int normed_proj(qasr_decoder* d, int rows, int n_out, const void* W, const f16* x, const void* nw,
                f16* y, const float* scale) {
    const int hs = d->cfg.hidden_size;
    const SkinnyShape sh = skinny_shape(d, rows, n_out, hs, scale != nullptr);
    if (norm_fusable(d, sh, hs, x))
        return launch_skinny<kOutF16, true>(
            d, sh, with_norm(d, skinny_args(d, sh, rows, n_out, hs, W, x, y, scale), nw));
    int rc = launch_rms_norm(x, hs, nw, d->n, rows, hs, d->ctx->cfg.rms_norm_eps, d->stream);
    if (rc) return rc;
    return gemm_f16(d, rows, n_out, hs, W, d->n, y, false, scale);
}

// logits[rows][vocab] (f32) = n[rows][hs] . E[vocab][hs]^T; with nw set,
// `nrows` are raw rows normed by gain nw first (in the kernel's prologue).
// *tile_cands is set when the skinny kernel also left each row's best
// (value, index) per column tile in am_v / am_i (argmax_tiles_kernel's input).
int gemm_logits(qasr_decoder* d, int rows, const f16* nrows, float* out, bool* tile_cands,
                const void* nw = nullptr) {
    const int hs = d->cfg.hidden_size, vocab = d->cfg.vocab_size;
    const SkinnyShape sh = skinny_shape(d, rows, vocab, hs);
    *tile_cands = false;
    if (sh.ks || sh.nks) {
        SkinnyArgs a = skinny_args(d, sh, rows, vocab, hs, d->embed, nrows, out);
        if (d->argmax_tiles && rows <= kSkinnyRows && vocab % 16 == 0) {
            a.am_v = d->am_v;
            a.am_i = d->am_i;
            *tile_cands = true;
            if (out == d->logits) a.Y = nullptr;  // no caller reads the scratch logits
        }
        if (nw) {
            if (!norm_fusable(d, sh, hs, nrows))
                return fail(QASR_EINVAL, "logits with a fused norm: not a skinny shape");
            return launch_skinny<kOutF32, true>(d, sh, with_norm(d, a, nw));
        }
        return launch_skinny<kOutF32>(d, sh, a);
    }
    if (nw) return fail(QASR_EINVAL, "logits with a fused norm: not a skinny shape");
    const float alpha = 1.0f, beta = 0.0f;
    const rocblas_status st = rocblas_gemm_ex(
        d->blas, rocblas_operation_transpose, rocblas_operation_none, vocab, rows, hs, &alpha,
        d->embed, rocblas_datatype_f16_r, hs, nrows, rocblas_datatype_f16_r, hs, &beta, out,
        rocblas_datatype_f32_r, vocab, out, rocblas_datatype_f32_r, vocab, rocblas_datatype_f32_r,
        rocblas_gemm_algo_standard, 0, 0);
    if (st != rocblas_status_success) return fail(QASR_EDEVICE, "rocblas_gemm_ex: %s", blas_msg(st));
    return QASR_OK;
}

int launch_rms_norm(const f16* x, int64_t x_stride, const void* w, f16* out, int rows, int hs,
                    float eps, hipStream_t st) {
    hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kNormThreads), 0, st, x, x_stride,
                       (const f16*)w, out, hs, eps);
    HIP_TRY(hipGetLastError(), "rms_norm launch");
    return QASR_OK;
}

// Everything after attention in one layer, then on to the next layer's input
// norm: o_proj + residual, post norm, gate|up, SiLU * up, down + residual.
int layer_tail(qasr_decoder* d, const qasr_layer_weights& L, int rows, hipStream_t st) {
    const qasr_attn_cfg& a = d->ctx->cfg;
    const int hs = d->cfg.hidden_size, inter = d->cfg.intermediate_size;
    const int qdim = a.num_attention_heads * a.head_dim;
    int rc = gemm_f16(d, rows, hs, qdim, L.o_proj, d->attn, d->x, true, L.o_scale);
    if (rc) return rc;
    // Post-attention norm folded into gate|up when it can be, else its own launch.
    bool fused = false;
    rc = glu_skinny(d, rows, inter, hs, L.gate_up_proj, d->x, d->h, L.gate_up_scale, L.post_norm,
                    &fused);
    if (rc) return rc;
    if (!fused) {
        rc = launch_rms_norm(d->x, hs, L.post_norm, d->n, rows, hs, a.rms_norm_eps, st);
        if (rc) return rc;
        rc = glu_skinny(d, rows, inter, hs, L.gate_up_proj, d->n, d->h, L.gate_up_scale, nullptr,
                        &fused);
        if (rc) return rc;
    }
    if (!fused) {
        rc = gemm_f16(d, rows, 2 * inter, hs, L.gate_up_proj, d->n, d->gu, false, L.gate_up_scale);
        if (rc) return rc;
        const int64_t threads = (int64_t)rows * (inter / 8);
        hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                           st, d->gu, inter, rows, d->h);
        HIP_TRY(hipGetLastError(), "silu_mul launch");
    }
    return gemm_f16(d, rows, hs, inter, L.down_proj, d->h, d->x, true, L.down_scale);
}

// Final norm of `rows` rows starting at x_rows, logits, argmax to next_dev;
// kHeadRows rows at a time.
int head(qasr_decoder* d, const f16* x_rows, int rows, int32_t* next_dev, float* logits_dev,
         hipStream_t st) {
    const int hs = d->cfg.hidden_size, vocab = d->cfg.vocab_size;
    for (int r0 = 0; r0 < rows; r0 += kHeadRows) {
        const int nr = std::min(kHeadRows, rows - r0);
        float* lg = logits_dev ? logits_dev + (int64_t)r0 * vocab : d->logits;
        int rc;
        bool tile_cands = false;
        if (r0 == 0 && norm_fusable(d, skinny_shape(d, nr, vocab, hs), hs, x_rows)) {
            rc = gemm_logits(d, nr, x_rows + (int64_t)r0 * hs, lg, &tile_cands, d->final_norm);  // norm folded
        } else {
            rc = launch_rms_norm(x_rows + (int64_t)r0 * hs, hs, d->final_norm, d->n, nr, hs,
                                 d->ctx->cfg.rms_norm_eps, st);
            if (rc) return rc;
            rc = gemm_logits(d, nr, d->n, lg, &tile_cands);
        }
        if (rc) return rc;
        if (tile_cands) {
            hipLaunchKernelGGL(argmax_tiles_kernel, dim3(nr), dim3(kArgTilesThreads), 0, st, d->am_v,
                               d->am_i, vocab / 16, vocab, next_dev + r0);
            HIP_TRY(hipGetLastError(), "argmax launch");
            continue;
        }
        hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgmaxChunks, nr), dim3(kArgmaxThreads), 0,
                           st, lg, vocab, d->am_v, d->am_i);
        HIP_TRY(hipGetLastError(), "argmax launch");
        hipLaunchKernelGGL(argmax_final_kernel, dim3(nr), dim3(64), 0, st, d->am_v, d->am_i, vocab,
                           next_dev + r0);
        HIP_TRY(hipGetLastError(), "argmax launch");
    }
    return QASR_OK;
}

int bind_stream(qasr_decoder* d, void* stream) {
    d->stream = (hipStream_t)stream;
    const char* e = std::getenv("QASR_DECODER_BLAS");
    d->force_blas = e && *e == '1';
    const char* f = std::getenv("QASR_DECODER_FUSE");
    d->fuse = !(f && *f == '0');
    const char* l = std::getenv("QASR_SKINNY_LDS");
    d->lds_gemm = l ? std::atoi(l) : 1;
    const char* tp = std::getenv("QASR_SKINNY_TPW");
    d->lds_tpw = tp ? std::atoi(tp) : 0;
    const char* gp = std::getenv("QASR_SKINNY_GROUPS");
    d->lds_groups = gp ? std::atoi(gp) : 0;
    const char* pg = std::getenv("QASR_PREFILL_GEMM");
    d->own_gemm = !(pg && std::string(pg) == "blas");
    const char* sh = std::getenv("QASR_SKINNY_SHARED");
    d->shared_tiles = sh ? std::atoi(sh) : 3;
    const char* mt = std::getenv("QASR_SKINNY_MULTI");
    d->multi_tiles = mt ? std::atoi(mt) : -1;
    const char* at = std::getenv("QASR_ARGMAX_TILES");
    d->argmax_tiles = !(at && *at == '0');
    const char* smt = std::getenv("QASR_SKINNY_SHARED_MIN_TILES");
    d->shared_min_tiles = smt ? std::atoi(smt) : 512;
    const rocblas_status st = rocblas_set_stream(d->blas, (hipStream_t)stream);
    if (st != rocblas_status_success) return fail(QASR_EDEVICE, "rocblas_set_stream: %s", blas_msg(st));
    return QASR_OK;
}

// Prefill of nseg segments whose hidden rows are concatenated in segment
// order: norms and projections once over all rows, stage (a) in one launch,
// attention per segment, then the head over each segment's last row.  Every
// argument is checked before the first launch.
int prefill_segments(qasr_decoder* dec, qasr_kv* kv, const qasr_segment* segs, int nseg,
                     const void* hidden_dev, int32_t* next_dev, float* logits_dev,
                     void* stream) {
    if (!dec || !kv) return fail(QASR_EINVAL, "null decoder or KV pool");
    if (kv->ctx != dec->ctx) return fail(QASR_EINVAL, "KV pool belongs to another context");
    if (!hidden_dev || !next_dev) return fail(QASR_EINVAL, "null argument");
    if (nseg > kMaxPrefillSegs)
        return fail(QASR_EINVAL, "%d segments in one prefill call, at most %d", nseg,
                    kMaxPrefillSegs);
    const qasr_ctx* ctx = dec->ctx;
    if (!ctx->cos) return fail(QASR_ESTATE, "RoPE tables not set (qasr_set_rope_tables)");
    int64_t total = 0;
    for (int i = 0; i < nseg; ++i) {
        const qasr_segment& g = segs[i];
        if (g.slot < 0 || g.slot >= kv->slots)
            return fail(QASR_EINVAL, "segment %d: slot %d outside [0, %d)", i, g.slot, kv->slots);
        if (g.pos0 < 0 || g.rows <= 0)
            return fail(QASR_EINVAL, "segment %d: kv_start %d / rows %d", i, g.pos0, g.rows);
        for (int j = 0; j < i; ++j)
            if (segs[j].slot == g.slot)
                return fail(QASR_EINVAL, "segments %d and %d share slot %d", j, i, g.slot);
        const int64_t end = (int64_t)g.pos0 + g.rows;
        if (end > ctx->cfg.max_seq)
            return fail(QASR_ERANGE, "prefill needs %lld positions, max_seq is %d",
                        (long long)end, ctx->cfg.max_seq);
        if (end > kv->cap)
            return fail(QASR_ERANGE, "prefill needs %lld positions, KV capacity is %d",
                        (long long)end, kv->cap);
        if (end > ctx->rope_rows)
            return fail(QASR_ERANGE, "prefill needs %lld positions, the RoPE tables hold %d",
                        (long long)end, ctx->rope_rows);
        total += g.rows;
    }
    if (total > dec->cfg.max_rows)
        return fail(QASR_EINVAL, "prefill rows %lld exceed max_rows %d", (long long)total,
                    dec->cfg.max_rows);
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    const hipStream_t st = (hipStream_t)stream;
    int rc = bind_stream(dec, stream);
    if (rc) return rc;
    const qasr_attn_cfg& a = ctx->cfg;
    const int hs = dec->cfg.hidden_size, rows = (int)total;
    const int qkvdim = (a.num_attention_heads + 2 * a.num_key_value_heads) * a.head_dim;
    HIP_TRY(hipMemcpyAsync(dec->x, hidden_dev, (size_t)rows * hs * 2, hipMemcpyDeviceToDevice, st),
            "prefill input copy");
    dec->ss_valid = false;
    // The layers' projections all take the GEMM, whatever the row count:
    // its per-element K order does not depend on how many rows (prompts)
    // share the launch, so a prompt's bits are those of its lone prefill.
    struct PrefillMode {
        qasr_decoder* d;
        explicit PrefillMode(qasr_decoder* dd) : d(dd) { d->prefill = true; }
        ~PrefillMode() { d->prefill = false; }
    };
    {
        PrefillMode mode(dec);
        for (int l = 0; l < a.num_hidden_layers; ++l) {
            const qasr_layer_weights& L = dec->layers[l];
            rc = normed_proj(dec, rows, qkvdim, L.qkv_proj, dec->x, L.input_norm, dec->qkv, L.qkv_scale);
            if (rc) return rc;
            rc = qasr_qk_norm_rope_append(dec->ctx, kv, l, segs, nseg, dec->qkv, L.q_norm, L.k_norm,
                                          dec->qw, stream);
            if (rc) return rc;
            rc = qasr_prefill_attn_batch(dec->ctx, kv, l, segs, nseg, dec->qw, dec->attn, stream);
            if (rc) return rc;
            rc = layer_tail(dec, L, rows, st);
            if (rc) return rc;
        }
    }
    if (nseg == 1) return head(dec, dec->x + (int64_t)(rows - 1) * hs, 1, next_dev, logits_dev, st);
    // Last rows into the gate|up scratch ([max_rows][2 inter], free after the
    // last layer; hs <= 2 inter is checked at creation), then the head.
    RowList last{};
    int64_t r0 = 0;
    for (int i = 0; i < nseg; ++i) {
        r0 += segs[i].rows;
        last.idx[i] = (int32_t)(r0 - 1);
    }
    hipLaunchKernelGGL(gather_rows_kernel, dim3(nseg), dim3(256), 0, st, dec->x, hs, last, dec->gu);
    HIP_TRY(hipGetLastError(), "row gather launch");
    return head(dec, dec->gu, nseg, next_dev, logits_dev, st);
}

// One decode step of `batch` (<= kSkinnyRows) rows, arguments checked.
int step_rows(qasr_decoder* dec, qasr_kv* kv, int batch, const int32_t* slots, const int32_t* pos,
              const int32_t* tokens_dev, int32_t* next_dev, float* logits_dev, hipStream_t st) {
    const qasr_attn_cfg& a = dec->ctx->cfg;
    const int hs = dec->cfg.hidden_size;
    const int qkvdim = (a.num_attention_heads + 2 * a.num_key_value_heads) * a.head_dim;
    // Chunk sums for a fused first norm when a skinny batch can use them.
    dec->ss_valid = dec->fuse && batch <= kSkinnyRows && hs <= kNormMaxK;
    hipLaunchKernelGGL(embed_rows_kernel, dim3(batch), dim3(256), 0, st, dec->embed, tokens_dev,
                       dec->cfg.vocab_size, hs, dec->x, dec->ss_valid ? dec->ss : nullptr);
    HIP_TRY(hipGetLastError(), "embedding launch");
    for (int l = 0; l < a.num_hidden_layers; ++l) {
        const qasr_layer_weights& L = dec->layers[l];
        int rc = normed_proj(dec, batch, qkvdim, L.qkv_proj, dec->x, L.input_norm, dec->qkv,
                             L.qkv_scale);
        if (rc) return rc;
        rc = qasr_decode_step(dec->ctx, kv, l, batch, slots, pos, dec->qkv, L.q_norm, L.k_norm,
                              dec->attn, st);
        if (rc) return rc;
        rc = layer_tail(dec, L, batch, st);
        if (rc) return rc;
    }
    return head(dec, dec->x, batch, next_dev, logits_dev, st);
}

}  // namespace

extern "C" {

int qasr_decoder_create(qasr_ctx* ctx, const qasr_decoder_cfg* cfg, const void* embed_dev,
                        const void* final_norm_dev, const qasr_layer_weights* layers,
                        qasr_decoder** out) {
    if (!out) return fail(QASR_EINVAL, "null output handle");
    *out = nullptr;
    if (!ctx || !cfg || !embed_dev || !final_norm_dev || !layers)
        return fail(QASR_EINVAL, "null argument");
    const qasr_attn_cfg& a = ctx->cfg;
    const int hs = cfg->hidden_size, inter = cfg->intermediate_size, vocab = cfg->vocab_size;
    if (hs <= 0 || hs % 8 || inter <= 0 || inter % 8 || vocab <= 0 || cfg->max_rows <= 0)
        return fail(QASR_EINVAL, "hidden %d / intermediate %d must be positive multiples of 8, "
                    "vocab %d and max_rows %d positive", hs, inter, vocab, cfg->max_rows);
    if (hs > 2 * inter)
        return fail(QASR_EINVAL, "hidden %d above 2 x intermediate %d", hs, inter);
    if (cfg->max_rows > kMaxDecoderRows)
        return fail(QASR_EINVAL, "max_rows %d above the limit of %d rows per call", cfg->max_rows,
                    kMaxDecoderRows);
    for (int l = 0; l < a.num_hidden_layers; ++l) {
        const qasr_layer_weights& L = layers[l];
        if (!L.input_norm || !L.qkv_proj || !L.q_norm || !L.k_norm || !L.o_proj || !L.post_norm ||
            !L.gate_up_proj || !L.down_proj)
            return fail(QASR_EINVAL, "layer %d: null weight pointer", l);
    }
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    qasr_decoder* d = new qasr_decoder;
    d->ctx = ctx;
    d->cfg = *cfg;
    d->embed = (const f16*)embed_dev;
    d->final_norm = (const f16*)final_norm_dev;
    d->layers.assign(layers, layers + a.num_hidden_layers);
    const size_t R = (size_t)cfg->max_rows;
    const size_t qdim = (size_t)a.num_attention_heads * a.head_dim;
    const size_t qkvdim = qdim + 2 * (size_t)a.num_key_value_heads * a.head_dim;
    // argmax candidates: the two-pass argmax's, or per column tile of the logits
    const size_t am_bytes = std::max((size_t)kHeadRows * kArgmaxChunks, (size_t)kSkinnyRows * (vocab / 16)) * 4;
    struct Alloc {
        void** p;
        size_t bytes;
    } allocs[] = {
        {(void**)&d->x, R * hs * 2},          {(void**)&d->n, R * hs * 2},
        {(void**)&d->qkv, R * qkvdim * 2},    {(void**)&d->qw, R * qdim * 2},
        {(void**)&d->attn, R * qdim * 2},     {(void**)&d->gu, R * 2 * (size_t)inter * 2},
        {(void**)&d->h, R * (size_t)inter * 2},
        {(void**)&d->logits, (size_t)kHeadRows * vocab * 4},
        {(void**)&d->am_v, am_bytes},
        {(void**)&d->am_i, am_bytes},
        {&d->blas_ws, kBlasWorkspace},
        {(void**)&d->sk_ws, (size_t)kSkinnyMaxTiles * kSkinnyMaxGroups * 1024},
        {(void**)&d->sk_ctr, (size_t)kSkinnyMaxTiles * 4},
        {(void**)&d->ss, (size_t)kSkinnyRows * kNormMaxChunks * 4},
    };
    // The largest int8 projection sets the prefill dequantisation scratch.
    int64_t wdq = 0;
    for (int l = 0; l < a.num_hidden_layers; ++l) {
        const qasr_layer_weights& L = layers[l];
        if (L.qkv_scale) wdq = std::max<int64_t>(wdq, (int64_t)qkvdim * hs);
        if (L.o_scale) wdq = std::max<int64_t>(wdq, (int64_t)hs * qdim);
        if (L.gate_up_scale) wdq = std::max<int64_t>(wdq, 2LL * inter * hs);
        if (L.down_scale) wdq = std::max<int64_t>(wdq, (int64_t)hs * inter);
    }
    if (wdq) {
        const hipError_t e = hipMalloc(&d->wdq, (size_t)wdq * 2);
        if (e != hipSuccess) {
            free_decoder(d);
            return hip_fail(e, "decoder dequantisation scratch");
        }
        d->wdq_elems = wdq;
    }
    for (const Alloc& al : allocs) {
        const hipError_t e = hipMalloc(al.p, al.bytes);
        if (e != hipSuccess) {
            free_decoder(d);
            return hip_fail(e, "decoder workspace");
        }
    }
    {
        const hipError_t e = hipMemset(d->sk_ctr, 0, (size_t)kSkinnyMaxTiles * 4);
        if (e != hipSuccess) {
            free_decoder(d);
            return hip_fail(e, "decoder counters");
        }
    }
    rocblas_status st = rocblas_create_handle(&d->blas);
    if (st == rocblas_status_success) st = rocblas_set_workspace(d->blas, d->blas_ws, kBlasWorkspace);
    if (st != rocblas_status_success) {
        free_decoder(d);
        return fail(QASR_EDEVICE, "rocBLAS handle: %s", blas_msg(st));
    }
    *out = d;
    return QASR_OK;
}

void qasr_decoder_destroy(qasr_decoder* dec) {
    if (!dec) return;
    DeviceScope ds(dec->ctx->device);
    (void)hipDeviceSynchronize();
    free_decoder(dec);
}

int qasr_decoder_step(qasr_decoder* dec, qasr_kv* kv, int batch, const int32_t* slots,
                      const int32_t* pos, const int32_t* tokens_dev, int32_t* next_dev,
                      float* logits_dev, void* stream) {
    if (!dec || !kv) return fail(QASR_EINVAL, "null decoder or KV pool");
    if (kv->ctx != dec->ctx) return fail(QASR_EINVAL, "KV pool belongs to another context");
    if (batch < 0 || batch > dec->cfg.max_rows)
        return fail(QASR_EINVAL, "batch %d outside [0, max_rows %d]", batch, dec->cfg.max_rows);
    if (batch == 0) return QASR_OK;
    if (!pos || !tokens_dev || !next_dev) return fail(QASR_EINVAL, "null argument");
    const qasr_ctx* ctx = dec->ctx;
    if (!ctx->cos) return fail(QASR_ESTATE, "RoPE tables not set (qasr_set_rope_tables)");
    // Every entry is checked before the first launch.
    std::vector<int32_t> sl(batch);
    std::vector<char> seen(kv->slots, 0);
    for (int b = 0; b < batch; ++b) {
        sl[b] = slots ? slots[b] : b;
        if (sl[b] < 0 || sl[b] >= kv->slots)
            return fail(QASR_EINVAL, "entry %d: slot %d outside [0, %d)", b, sl[b], kv->slots);
        if (seen[sl[b]]++) return fail(QASR_EINVAL, "entry %d: slot %d appears twice", b, sl[b]);
        if (pos[b] < 0) return fail(QASR_EINVAL, "entry %d: negative position", b);
        if (pos[b] >= kv->cap)
            return fail(QASR_ERANGE, "entry %d: position %d beyond KV capacity %d", b, pos[b], kv->cap);
        if (pos[b] >= ctx->cfg.max_seq)
            return fail(QASR_ERANGE, "entry %d: decode past max_seq %d", b, ctx->cfg.max_seq);
        if (pos[b] >= ctx->rope_rows)
            return fail(QASR_ERANGE, "entry %d: position %d beyond the %d RoPE table rows", b,
                        pos[b], ctx->rope_rows);
    }
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    int rc = bind_stream(dec, stream);
    if (rc) return rc;
    // Batches past kSkinnyRows rows run as consecutive groups of at most
    // kSkinnyRows rows: every projection then runs the kernels of a lone
    // slot's step, so each slot's bits are those of its step alone (the
    // reference's --batch N == --batch 1).  The weights are read once per group.
    const int64_t vocab = dec->cfg.vocab_size;
    for (int b0 = 0; b0 < batch; b0 += kSkinnyRows) {
        const int nb = std::min(kSkinnyRows, batch - b0);
        rc = step_rows(dec, kv, nb, sl.data() + b0, pos + b0, tokens_dev + b0, next_dev + b0,
                       logits_dev ? logits_dev + b0 * vocab : nullptr, (hipStream_t)stream);
        if (rc) return rc;
    }
    return QASR_OK;
}

int qasr_decoder_prefill(qasr_decoder* dec, qasr_kv* kv, int slot, int kv_start, int s,
                         const void* hidden_dev, int32_t* next_dev, float* logits_dev,
                         void* stream) {
    const qasr_segment seg{slot, kv_start, s};
    return prefill_segments(dec, kv, &seg, 1, hidden_dev, next_dev, logits_dev, stream);
}

int qasr_decoder_prefill_batch(qasr_decoder* dec, qasr_kv* kv, const qasr_segment* segs,
                               int nseg, const void* hidden_dev, int32_t* next_dev,
                               float* logits_dev, void* stream) {
    if (nseg < 0 || (nseg > 0 && !segs)) return fail(QASR_EINVAL, "bad segment list");
    if (nseg == 0) return QASR_OK;
    return prefill_segments(dec, kv, segs, nseg, hidden_dev, next_dev, logits_dev, stream);
}

int qasr_gemm_f16(qasr_ctx* ctx, const void* a_dev, const void* b_dev, void* c_dev, int32_t m,
                  int32_t n, int32_t k, int accumulate, void* stream) {
    if (!ctx) return fail(QASR_EINVAL, "null context");
    if (m < 0 || n < 0 || k < 0) return fail(QASR_EINVAL, "negative GEMM size %d x %d x %d", m, n, k);
    if (m == 0 || n == 0) return QASR_OK;
    if (!qasr::gemm_f16_fits(m, n, k))
        return fail(QASR_EINVAL, "GEMM %d x %d x %d: k must be a positive multiple of 64, n of 256, "
                    "and each operand under 2 GB", m, n, k);
    if (!a_dev || !b_dev || !c_dev) return fail(QASR_EINVAL, "null device pointer");
    if ((uintptr_t)a_dev % 16 || (uintptr_t)b_dev % 16 || (uintptr_t)c_dev % 16)
        return fail(QASR_EINVAL, "a, b and c must be 16-byte aligned");
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    HIP_TRY(qasr::launch_gemm_f16((const f16*)a_dev, (const f16*)b_dev, (f16*)c_dev, m, n, k,
                                  accumulate != 0, ctx->cus, (hipStream_t)stream),
            "GEMM launch");
    return QASR_OK;
}

int qasr_dequant_i8(qasr_ctx* ctx, const void* q_dev, const float* scale_dev, int64_t rows,
                    int32_t cols, void* out_dev, void* stream) {
    if (!ctx) return fail(QASR_EINVAL, "null context");
    if (rows < 0 || cols < 0 || cols % 8)
        return fail(QASR_EINVAL, "int8 matrix %lld x %d: cols must be a multiple of 8",
                    (long long)rows, cols);
    if (rows == 0 || cols == 0) return QASR_OK;
    if (!q_dev || !scale_dev || !out_dev) return fail(QASR_EINVAL, "null device pointer");
    if ((uintptr_t)q_dev % 8 || (uintptr_t)out_dev % 16)
        return fail(QASR_EINVAL, "q must be 8-byte and out 16-byte aligned");
    const int64_t groups8 = rows * cols / 8;
    if ((groups8 + 255) / 256 > (int64_t)UINT32_MAX)
        return fail(QASR_EINVAL, "int8 matrix of %lld elements is too large", (long long)(rows * cols));
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    hipLaunchKernelGGL(dequant_rows_kernel, dim3((unsigned)((groups8 + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const int8_t*)q_dev, scale_dev, rows, (int)cols,
                       (f16*)out_dev);
    HIP_TRY(hipGetLastError(), "dequantisation launch");
    return QASR_OK;
}

}  // extern "C"
