// decode_attn.hip -- stage (b): GQA decode attention over ragged per-slot
// contexts, split-K with an in-kernel merge; optionally fused with stage (a).
//
// Replaces the reference's gqa_decode_single[_slots], gqa_decode_split_p1_pair
// and gqa_split_merge (src/shaders.rs:1881-2905, planned in src/decoder.rs:
// 1932-2025 and 3348-3451).  Semantics: src/cpu_decoder.rs:292-365 with one
// query row, i.e. softmax(q.k_t * scale) . v over keys t < cur_len.
//
// Work decomposition (one launch for the whole batch):
//   workgroup = (batch entry b, kv head, chunk of `chunk` keys), 4 waves.
//   Both q heads of the kv head (GQA 2:1) are computed from one K/V read.
//   A wave pass covers 32 keys: 8 dwordx4 loads of K and 8 of V per lane, each
//   load instruction reading 1 KiB contiguous (4 keys x 256 B, lane l -> key
//   l/16, dims (l%16)*8..+8), so every instruction is fully coalesced.  Keys
//   past the chunk end load a clamped (valid) row and are masked to -inf.
//   The next pass's K loads are issued right after this pass's scores, and its
//   V loads right after this pass's P.V, so memory stays busy during compute.
//   q.k: v_dot2_f32_f16 on the lane's 8 dims, then a 16-lane DPP all-reduce
//   inside the row (no LDS).  Softmax is online per 16-lane row (exp2 domain),
//   P.V accumulates in f32 registers (v_fma_mix).  Rows and waves merge through
//   LDS.  When an entry needs more than one chunk, each workgroup publishes
//   its partial (max, sum, unnormalised output) with device-scope stores and
//   the last one to arrive (ticket) merges them: no second launch and no
//   L2-wide cache maintenance.
//
// Fused variant (stage (a) + (b)): the workgroup recomputes its two q heads
// from the raw qkv row (bit-identical to the stage-(a) kernel); the workgroup
// owning the last chunk also ropes the new K row, appends K and V to the cache
// and substitutes them for the cache load of that key.  The first K/V pass is
// issued before this prologue so its latency overlaps it.

#include "kernels.hpp"
#include "norm_rope.hpp"

namespace qasr {

namespace {

__device__ __forceinline__ float dot8(const H8& a, const H8& b) {
    float s = 0.0f;
    s = __builtin_amdgcn_fdot2(a.h2[0], b.h2[0], s, false);
    s = __builtin_amdgcn_fdot2(a.h2[1], b.h2[1], s, false);
    s = __builtin_amdgcn_fdot2(a.h2[2], b.h2[2], s, false);
    s = __builtin_amdgcn_fdot2(a.h2[3], b.h2[3], s, false);
    return s;
}

constexpr float kNegInf = -__builtin_inff();

// One wave pass of 8 loads (32 keys) of K or V starting at key t0; keys at or
// past `kend` are clamped to row kend-1 (valid, masked later).
__device__ __forceinline__ void load_pass(const f16* __restrict__ base, int t0, int kend, int row,
                                          int seg, H8 (&r)[8]) {
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
        const int key = min(t0 + kk * 4 + row, kend - 1);
        r[kk].u = *(const uint4*)(base + (int64_t)key * kHeadDim + seg * 8);
    }
}

template <bool FUSED>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_attn_kernel(
    CacheGeom g, int layer, DecodePlan P, const f16* __restrict__ qin,
    const f16* __restrict__ q_gain, const f16* __restrict__ k_gain,
    const f16* __restrict__ cos_tab, const f16* __restrict__ sin_tab, f16* __restrict__ out,
    float* __restrict__ ws_acc, float* __restrict__ ws_ml, uint32_t* __restrict__ counters) {
    constexpr int kRows = kDecodeWaves * 4;  // 16-lane rows per workgroup
    __shared__ H8 s_q[2][16];
    __shared__ H8 s_knew[16];
    __shared__ H8 s_vnew[16];
    __shared__ __attribute__((aligned(16))) f16 s_raw[4][kHeadDim];  // q0, q1, k, v raw heads
    __shared__ __attribute__((aligned(16))) f16 s_tab[4][kHeadDim];  // q gain, k gain, cos, sin
    __shared__ float s_inv[3];
    __shared__ float s_m[kRows][2];
    __shared__ float s_l[kRows][2];
    __shared__ float s_acc[kRows][2][kHeadDim];
    __shared__ int s_last;

    const int wg = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int row = lane >> 4;  // key within a 4-key load
    const int seg = lane & 15;  // 8-dim segment

    int b = 0;
    {
        int lo = 0, hi = P.batch - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (P.wg_base[mid] <= wg) lo = mid; else hi = mid - 1;
        }
        b = lo;
    }
    const int L = P.len[b];
    const int nch = (L + P.chunk - 1) / P.chunk;
    const int rel = wg - P.wg_base[b];
    const int kvh = rel / nch;
    const int c = rel - kvh * nch;
    const int key0 = c * P.chunk;
    const int key1 = min(key0 + P.chunk, L);
    const int nqh = P.nqh;
    const int h0 = kvh * kRep;
    f16* Kc = g.base + P.slot[b] * g.slot_stride + layer * g.layer_stride + kvh * g.head_stride;
    f16* Vc = Kc + g.kv_stride;

    // Raw inputs of the fused prologue are requested before the first K/V pass
    // so that waiting for them does not wait for the pass.
    const int pos = L - 1;
    const bool owner = FUSED && (c == nch - 1);
    if constexpr (FUSED) {
        const int64_t tot = (int64_t)(nqh + 2 * g.nkvh) * kHeadDim;
        const f16* qkv_row = qin + b * tot;
        if (tid < 64) {
            const int which = tid >> 4;
            const int hoff = which < 2 ? (h0 + which) : which == 2 ? (nqh + kvh) : (nqh + g.nkvh + kvh);
            *(uint4*)&s_raw[which][seg * 8] = *(const uint4*)(qkv_row + hoff * kHeadDim + seg * 8);
        } else if (tid < 128) {
            const int which = (tid >> 4) & 3;
            const f16* p = which == 0 ? q_gain
                         : which == 1 ? k_gain
                         : which == 2 ? cos_tab + (int64_t)pos * kHeadDim
                                      : sin_tab + (int64_t)pos * kHeadDim;
            *(uint4*)&s_tab[which][seg * 8] = *(const uint4*)(p + seg * 8);
        }
    }

    H8 kr[8], vr[8];
    int t0 = key0 + wave * kDecodeTileKeys;
    load_pass(Kc, t0, key1, row, seg, kr);
    load_pass(Vc, t0, key1, row, seg, vr);

    H8 q0, q1;
    if constexpr (FUSED) {
        __syncthreads();
        if (tid < 3 && (tid < 2 || owner)) s_inv[tid] = head_inv_rms_serial(s_raw[tid], P.eps);
        __syncthreads();
        const int h = tid >> 7, j = tid & 127;
        ((f16*)s_q[h])[j] = rope_elem(s_raw[h], s_tab[0], s_tab[2], s_tab[3], s_inv[h], j);
        if (owner) {
            if (h == 0) {
                const f16 kv = rope_elem(s_raw[2], s_tab[1], s_tab[2], s_tab[3], s_inv[2], j);
                ((f16*)s_knew)[j] = kv;
                Kc[(int64_t)pos * kHeadDim + j] = kv;
            } else {
                const f16 vv = s_raw[3][j];
                ((f16*)s_vnew)[j] = vv;
                Vc[(int64_t)pos * kHeadDim + j] = vv;
            }
        }
        __syncthreads();
        q0 = s_q[0][seg];
        q1 = s_q[1][seg];
    } else {
        const f16* qb = qin + (int64_t)b * nqh * kHeadDim + h0 * kHeadDim + seg * 8;
        q0.u = *(const uint4*)qb;
        q1.u = *(const uint4*)(qb + kHeadDim);
    }

    float m0 = kNegInf, m1 = kNegInf, l0 = 0.0f, l1 = 0.0f;
    float a0[8], a1[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) a0[d] = a1[d] = 0.0f;

    const float sl2 = P.scale_log2;
    for (; t0 < key1; t0 += kDecodeWgKeys) {
        if constexpr (FUSED) {
            if (owner) {
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    if (t0 + kk * 4 + row == pos) {
                        kr[kk] = s_knew[seg];
                        vr[kk] = s_vnew[seg];
                    }
                }
            }
        }
        float s0[8], s1[8];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            s0[kk] = row_sum16(dot8(q0, kr[kk])) * sl2;
            s1[kk] = row_sum16(dot8(q1, kr[kk])) * sl2;
            if (t0 + kk * 4 + row >= key1) s0[kk] = s1[kk] = kNegInf;
        }
        const int tn = t0 + kDecodeWgKeys;
        if (tn < key1) load_pass(Kc, tn, key1, row, seg, kr);
        float mt0 = s0[0], mt1 = s1[0];
#pragma unroll
        for (int kk = 1; kk < 8; ++kk) {
            mt0 = fmaxf(mt0, s0[kk]);
            mt1 = fmaxf(mt1, s1[kk]);
        }
        const float mn0 = fmaxf(m0, mt0), mn1 = fmaxf(m1, mt1);
        const float mu0 = mn0 == kNegInf ? 0.0f : mn0;
        const float mu1 = mn1 == kNegInf ? 0.0f : mn1;
        const float al0 = fast_exp2(m0 - mu0), al1 = fast_exp2(m1 - mu1);
        m0 = mn0;
        m1 = mn1;
        float ps0 = 0.0f, ps1 = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            s0[kk] = fast_exp2(s0[kk] - mu0);
            s1[kk] = fast_exp2(s1[kk] - mu1);
            ps0 += s0[kk];
            ps1 += s1[kk];
        }
        l0 = l0 * al0 + ps0;
        l1 = l1 * al1 + ps1;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            a0[d] *= al0;
            a1[d] *= al1;
        }
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                const float v = h2f(vr[kk].e[d]);
                a0[d] = fmaf(s0[kk], v, a0[d]);
                a1[d] = fmaf(s1[kk], v, a1[d]);
            }
        }
        if (tn < key1) load_pass(Vc, tn, key1, row, seg, vr);
    }

    // Merge the 16 rows of the workgroup (each row saw a disjoint key subset).
    const int r16 = wave * 4 + row;
    if (seg == 0) {
        s_m[r16][0] = m0;
        s_m[r16][1] = m1;
        s_l[r16][0] = l0;
        s_l[r16][1] = l1;
    }
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        s_acc[r16][0][seg * 8 + d] = a0[d];
        s_acc[r16][1][seg * 8 + d] = a1[d];
    }
    __syncthreads();
    const int h = tid >> 7, j = tid & 127;
    float M = kNegInf;
#pragma unroll
    for (int r = 0; r < kRows; ++r) M = fmaxf(M, s_m[r][h]);
    float Ls = 0.0f, A = 0.0f;
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const float mr = s_m[r][h];
        const float w = mr == kNegInf ? 0.0f : fast_exp2(mr - M);
        Ls = fmaf(s_l[r][h], w, Ls);
        A = fmaf(s_acc[r][h][j], w, A);
    }
    f16* ob = out + (int64_t)b * nqh * kHeadDim + (h0 + h) * kHeadDim + j;
    if (nch == 1) {
        *ob = f2h(A / Ls);
        return;
    }

    store_dev(&ws_acc[(int64_t)wg * (2 * kHeadDim) + h * kHeadDim + j], A);
    if (j == 0) {
        store_dev(&ws_ml[(int64_t)wg * 4 + h], M);
        store_dev(&ws_ml[(int64_t)wg * 4 + 2 + h], Ls);
    }
    stores_done_barrier();
    uint32_t* ctr = &counters[b * g.nkvh + kvh];
    if (tid == 0) s_last = (ticket_add(ctr) == (uint32_t)(nch - 1));
    __syncthreads();
    if (!s_last) return;
    const int64_t it0 = P.wg_base[b] + kvh * nch;
    float M2 = kNegInf;
    for (int i = 0; i < nch; ++i) M2 = fmaxf(M2, load_dev(&ws_ml[(it0 + i) * 4 + h]));
    float L2 = 0.0f, A2 = 0.0f;
    for (int i = 0; i < nch; ++i) {
        const float mi = load_dev(&ws_ml[(it0 + i) * 4 + h]);
        const float w = mi == kNegInf ? 0.0f : fast_exp2(mi - M2);
        L2 = fmaf(load_dev(&ws_ml[(it0 + i) * 4 + 2 + h]), w, L2);
        A2 = fmaf(load_dev(&ws_acc[(it0 + i) * (2 * kHeadDim) + h * kHeadDim + j]), w, A2);
    }
    *ob = f2h(A2 / L2);
    if (tid == 0) ticket_reset(ctr);
}

}  // namespace

hipError_t launch_decode_attn(bool fused, const CacheGeom& g, int layer, const DecodePlan& P,
                              int total_wgs, const f16* q_or_qkv, const f16* q_gain,
                              const f16* k_gain, const f16* cos_tab, const f16* sin_tab,
                              f16* out, const DecodeWs& ws, hipStream_t stream) {
    if (total_wgs <= 0) return hipSuccess;
    if (total_wgs > ws.items) return hipErrorInvalidValue;
    const dim3 grid(total_wgs), block(kDecodeWaves * 64);
    if (fused)
        hipLaunchKernelGGL(decode_attn_kernel<true>, grid, block, 0, stream, g, layer, P, q_or_qkv,
                           q_gain, k_gain, cos_tab, sin_tab, out, ws.acc, ws.ml, ws.counters);
    else
        hipLaunchKernelGGL(decode_attn_kernel<false>, grid, block, 0, stream, g, layer, P,
                           q_or_qkv, q_gain, k_gain, cos_tab, sin_tab, out, ws.acc, ws.ml,
                           ws.counters);
    return hipGetLastError();
}

}  // namespace qasr
