// decode_attn.hip -- stage (b): GQA decode attention over ragged per-slot
// contexts, split-K with an in-kernel merge; optionally fused with stage (a).
//
// Replaces the reference's gqa_decode_single[_slots], gqa_decode_split_p1_pair
// and gqa_split_merge (src/shaders.rs:1881-2905, planned in src/decoder.rs:
// 1932-2025 and 3348-3451).  Semantics: src/cpu_decoder.rs:292-365 with one
// query row, i.e. softmax(q.k_t * scale) . v over keys t < cur_len.
//
// Work decomposition (one launch for the whole batch):
//   workgroup = (batch entry b, kv head, chunk of keys), W waves.  Chunk sizes
//   are planned per entry on the host so every workgroup streams about the
//   same number of keys whatever the ragged lengths.
//   Both q heads of the kv head (GQA 2:1) are computed from one K/V read.
//   A wave pass covers 32 contiguous keys (wave w of a workgroup pass takes
//   keys t0 + 32*w .. +32, so the workgroup's requests of one pass form one
//   contiguous run): 8 dwordx4 buffer loads of K and 8 of V per lane, each
//   instruction reading 1 KiB contiguous (4 keys x 256 B, lane l -> key l/16,
//   dims (l%16)*8..+8), so every instruction is fully coalesced.  (Spreading
//   a wave's loads over the workgroup pass in 4-key groups, or giving each
//   wave one contiguous share of the chunk, both measured slower.)
//   The buffer resources end at the chunk's last key, so the hardware range
//   check returns zeros past it (those scores are masked).
//   q.k: v_dot2_f32_f16 on the lane's 8 dims, then a transposing 16-lane DPP
//   reduction that leaves each lane with one (key, head) score.  Softmax is
//   online per (16-lane row, head) in the exp2 domain; the row's 16
//   probabilities reach the V layout through LDS and P.V accumulates in f32
//   (v_fma_mix on packed f16).  The 4W rows of the workgroup merge through
//   one LDS pass.
//   When an entry needs more than one chunk, each workgroup publishes its
//   partial (max, sum, unnormalised output) with device-scope stores and the
//   last one to arrive (ticket) merges them, issuing all its loads at once:
//   no second launch and no L2-wide cache maintenance.
//
// Fused variant (stage (a) + (b)): the workgroup recomputes its two q heads
// from the raw qkv row (bit-identical to the stage-(a) kernel); the workgroup
// owning the last chunk also ropes the new K row, appends K and V to the cache
// and substitutes them for the cache load of that key.  The first K/V pass is
// issued before this prologue so its latency overlaps it.

#include <type_traits>

#include "kernels.hpp"
#include "norm_rope.hpp"

namespace qasr {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kNegInf = -__builtin_inff();
constexpr int kSc1 = 16;  // buffer cache policy: sc1 (device-coherent, as agent-scope atomics)
// Buffer cache policy nt (non-temporal) for the K/V stream: each byte is read
// once per launch, and streaming it with the default policy measured 7-9%
// slower (config 3: 23.3 against 21.7 us; 16 x 2048 keys: 29.2 against 26.5).
constexpr int kNt = 2;

__device__ __forceinline__ float dot8(const H8& a, const H8& b) {
    float s = 0.0f;
    s = __builtin_amdgcn_fdot2(a.h2[0], b.h2[0], s, false);
    s = __builtin_amdgcn_fdot2(a.h2[1], b.h2[1], s, false);
    s = __builtin_amdgcn_fdot2(a.h2[2], b.h2[2], s, false);
    s = __builtin_amdgcn_fdot2(a.h2[3], b.h2[3], s, false);
    return s;
}

// Buffer resource over `bytes` bytes at `p` (raw buffer, gfx9 data format).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// One wave pass (32 keys from t0) of K or V: 8 x 16 B per lane; load kk
// covers keys t0 + 4*kk .. +4 (this lane: key t0 + 4*kk + row).  Non-temporal.
__device__ __forceinline__ void load_pass(__amdgpu_buffer_rsrc_t r, int t0, int row, int seg,
                                          H8 (&x)[8]) {
    const int voff = (t0 + row) * (kHeadDim * 2) + seg * 16;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff + kk * 1024, 0, kNt);
        x[kk].u = make_uint4(v.x, v.y, v.z, v.w);
    }
}

template <bool FUSED, int W>
__global__ __launch_bounds__(W * 64)
__attribute__((amdgpu_waves_per_eu(kDecodeWavesPerEU, 8))) void decode_attn_kernel(
    CacheGeom g, int layer, DecodePlan P, const f16* __restrict__ qin,
    const f16* __restrict__ q_gain, const f16* __restrict__ k_gain,
    const f16* __restrict__ cos_tab, const f16* __restrict__ sin_tab, f16* __restrict__ out,
    float* __restrict__ ws_acc, float* __restrict__ ws_ml, uint32_t* __restrict__ counters) {
    __shared__ H8 s_q[2][16];
    __shared__ H8 s_knew[16];
    __shared__ H8 s_vnew[16];
    __shared__ __attribute__((aligned(16))) f16 s_raw[4][kHeadDim];  // q0, q1, k, v raw heads
    __shared__ __attribute__((aligned(16))) f16 s_tab[4][kHeadDim];  // q gain, k gain, cos, sin
    __shared__ __attribute__((aligned(16))) float s_sq[3][kHeadDim];  // squares of q0, q1, k
    __shared__ float s_inv[3];
    __shared__ float s_p[W][64];
    __shared__ float s_wm[4 * W][2];
    __shared__ float s_wl[4 * W][2];
    __shared__ float s_wa[4 * W][2][kHeadDim];
    __shared__ int s_last;

    const int wg = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int row = lane >> 4;  // key within a 4-key load
    const int seg = lane & 15;  // 8-dim segment

    // Entry of this workgroup = number of later entry starts at or before it:
    // lane i tests wg_base[i + 1], one load per lane and a ballot, no search.
    static_assert(kMaxBatch <= 64, "one lane per entry");
    const int b = __popcll(__ballot(lane + 1 < P.batch && P.wg_base[lane + 1] <= wg));
    const int L = P.len[b];
    const int chunk = P.chunk[b];
    const int nch = (L + chunk - 1) / chunk;
    const int rel = wg - P.wg_base[b];
    const int kvh = rel / nch;
    const int c = rel - kvh * nch;
    const int key0 = c * chunk;
    const int key1 = min(key0 + chunk, L);
    const int nkeys = key1 - key0;
    const int nqh = P.nqh;
    const int h0 = kvh * kRep;
    f16* Kc = g.base + P.slot[b] * g.slot_stride + layer * g.layer_stride + kvh * g.head_stride;
    f16* Vc = Kc + g.kv_stride;
    // Resources start at the chunk's first key and end at its last.
    const int rbytes = nkeys * (kHeadDim * 2);
    const __amdgpu_buffer_rsrc_t kres = make_rsrc(Kc + (int64_t)key0 * kHeadDim, rbytes);
    const __amdgpu_buffer_rsrc_t vres = make_rsrc(Vc + (int64_t)key0 * kHeadDim, rbytes);
    constexpr int kWgKeys = W * kDecodeTileKeys;  // keys per workgroup pass
    const int tw = wave * kDecodeTileKeys;         // this wave's first key in a pass

    // The query inputs (the raw qkv heads, or q itself) are requested first and
    // the first K/V pass right after them, so the K/V stream starts without
    // waiting for a round trip; the prologue runs while the pass is in flight.
    const int pos = L - 1;
    const bool owner = FUSED && (c == nch - 1);
    H8 q0, q1;
    if constexpr (FUSED) {
        const int64_t tot = (int64_t)(nqh + 2 * g.nkvh) * kHeadDim;
        const f16* qkv_row = qin + b * tot;
        if (tid < 64) {
            const int which = tid >> 4;
            const int hoff = which < 2 ? (h0 + which) : which == 2 ? (nqh + kvh) : (nqh + g.nkvh + kvh);
            H8 x;
            x.u = *(const uint4*)(qkv_row + hoff * kHeadDim + seg * 8);
            *(uint4*)&s_raw[which][seg * 8] = x.u;
            if (which < 3) {  // f16 squares are exact in f32
                float4 lo, hi;
                lo.x = h2f(x.e[0]) * h2f(x.e[0]);
                lo.y = h2f(x.e[1]) * h2f(x.e[1]);
                lo.z = h2f(x.e[2]) * h2f(x.e[2]);
                lo.w = h2f(x.e[3]) * h2f(x.e[3]);
                hi.x = h2f(x.e[4]) * h2f(x.e[4]);
                hi.y = h2f(x.e[5]) * h2f(x.e[5]);
                hi.z = h2f(x.e[6]) * h2f(x.e[6]);
                hi.w = h2f(x.e[7]) * h2f(x.e[7]);
                *(float4*)&s_sq[which][seg * 8] = lo;
                *(float4*)&s_sq[which][seg * 8 + 4] = hi;
            }
        } else if (tid < 128) {
            const int which = (tid >> 4) & 3;
            const f16* p = which == 0 ? q_gain
                         : which == 1 ? k_gain
                         : which == 2 ? cos_tab + (int64_t)pos * kHeadDim
                                      : sin_tab + (int64_t)pos * kHeadDim;
            *(uint4*)&s_tab[which][seg * 8] = *(const uint4*)(p + seg * 8);
        }
    } else {
        const f16* qb = qin + (int64_t)b * nqh * kHeadDim + h0 * kHeadDim + seg * 8;
        q0.u = *(const uint4*)qb;
        q1.u = *(const uint4*)(qb + kHeadDim);
    }

    // Two pass buffers per wave: while one pass is computed the next one's
    // loads are in flight.  Passes past the chunk fall outside the buffer
    // range: their loads return zeros without touching memory.
    H8 ka[8], va[8], kb[8], vb[8];
    load_pass(kres, tw, row, seg, ka);
    load_pass(vres, tw, row, seg, va);

    if constexpr (FUSED) {
        __syncthreads();
        if (tid < 3 && (tid < 2 || owner)) s_inv[tid] = head_inv_rms_squares(s_sq[tid], P.eps);
        __syncthreads();
        if (tid < 256) {
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
        }
        __syncthreads();
        q0 = s_q[0][seg];
        q1 = s_q[1][seg];
    }

    load_pass(kres, tw + kWgKeys, row, seg, kb);
    load_pass(vres, tw + kWgKeys, row, seg, vb);

    // Per 16-lane row: running (max, sum) of the head given by the lane's
    // parity (replicated over the 8 lanes of that parity), and the lane's 8
    // output dims of both heads.
    float m_run = kNegInf, l_run = 0.0f;
    float a0[8], a1[8];
#pragma unroll
    for (int d = 0; d < 8; ++d) a0[d] = a1[d] = 0.0f;
    const bool odd = seg & 1;
    float* s_pw = &s_p[wave][0];
    const float sl2 = P.scale_log2;
    const int new_rel = pos - key0;  // the appended key, relative to the chunk (owner only)

    auto process = [&](H8 (&kr)[8], H8 (&vr)[8], int t0) {
        if constexpr (FUSED) {
            if (owner) {
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    if (t0 + 4 * kk + row == new_rel) {
                        kr[kk] = s_knew[seg];
                        vr[kk] = s_vnew[seg];
                    }
                }
            }
        }
        // Partial dots of the lane's 8 dims, value index kk*2 + head; the
        // transposing row reduction leaves lane seg of row `row` with the full
        // score of key t0 + 4*(seg>>1) + row, head seg&1.
        float v[16];
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            v[2 * kk] = dot8(q0, kr[kk]);
            v[2 * kk + 1] = dot8(q1, kr[kk]);
        }
        const float sc = row_reduce_transpose16(v, seg);
        const int my_key = t0 + 4 * (seg >> 1) + row;
        const float sv = my_key < nkeys ? sc * sl2 : kNegInf;
        // Online softmax per (row, head): max / sum over the 8 lanes of the
        // lane's parity.
        float mt = fmaxf(sv, dpp<kDppXor2>(sv));
        mt = fmaxf(mt, dpp<kDppRor4>(mt));
        mt = fmaxf(mt, dpp<kDppRor8>(mt));
        const float mn = fmaxf(m_run, mt);
        const float mu = mn == kNegInf ? 0.0f : mn;
        const float alpha = softmax_w_scaled(m_run, mu);
        const float pv = softmax_w_scaled(sv, mu);
        m_run = mn;
        float ps = pv + dpp<kDppXor2>(pv);
        ps += dpp<kDppRor4>(ps);
        ps += dpp<kDppRor8>(ps);
        l_run = l_run * alpha + ps;
        // Broadcast the row's 16 probabilities to the V layout through LDS.
        s_pw[lane] = pv;
        const float alpha_x = dpp<kDppXor1>(alpha);  // the other head's factor
        const float al0 = odd ? alpha_x : alpha, al1 = odd ? alpha : alpha_x;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            a0[d] *= al0;
            a1[d] *= al1;
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
            const float2 p2 = *(const float2*)&s_pw[16 * row + 2 * kk];
            const uint32_t w4[4] = {vr[kk].u.x, vr[kk].u.y, vr[kk].u.z, vr[kk].u.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                fma_mix_lo(a0[2 * e], p2.x, w4[e]);
                fma_mix_lo(a1[2 * e], p2.y, w4[e]);
                fma_mix_hi(a0[2 * e + 1], p2.x, w4[e]);
                fma_mix_hi(a1[2 * e + 1], p2.y, w4[e]);
            }
        }
        __builtin_amdgcn_wave_barrier();
    };

    for (int t0 = tw; t0 < nkeys; t0 += 2 * kWgKeys) {
        process(ka, va, t0);
        __builtin_amdgcn_sched_barrier(0);
        load_pass(kres, t0 + 2 * kWgKeys, row, seg, ka);
        load_pass(vres, t0 + 2 * kWgKeys, row, seg, va);
        if (t0 + kWgKeys < nkeys) process(kb, vb, t0 + kWgKeys);
        __builtin_amdgcn_sched_barrier(0);
        load_pass(kres, t0 + 3 * kWgKeys, row, seg, kb);
        load_pass(vres, t0 + 3 * kWgKeys, row, seg, vb);
    }

    // Merge the 4W rows of the workgroup through LDS: every row holds the
    // (max, sum) of the head of the lane's parity and 8 dims of both heads.
    {
        const int r = wave * 4 + row;
        if (seg < 2) {  // lane 0 of the row holds head 0's (m, l), lane 1 head 1's
            s_wm[r][seg] = m_run;
            s_wl[r][seg] = l_run;
        }
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            s_wa[r][0][seg * 8 + d] = a0[d];
            s_wa[r][1][seg * 8 + d] = a1[d];
        }
    }
    __syncthreads();
    if (tid >= 256) return;  // 256 threads: one per (head, dim)
    const int h = tid >> 7, j = tid & 127;
    float M = kNegInf;
#pragma unroll
    for (int r = 0; r < 4 * W; ++r) M = fmaxf(M, s_wm[r][h]);
    float Ls = 0.0f, A = 0.0f;
#pragma unroll
    for (int r = 0; r < 4 * W; ++r) {
        const float mr = s_wm[r][h];
        const float f = mr == kNegInf ? 0.0f : fast_exp2(mr - M);
        Ls = fmaf(s_wl[r][h], f, Ls);
        A = fmaf(s_wa[r][h][j], f, A);
    }
    f16* ob = out + (int64_t)b * nqh * kHeadDim + h0 * kHeadDim;
    if (nch == 1) {
        ob[h * kHeadDim + j] = f2h(A / Ls);
        return;
    }

    store_dev(&ws_acc[(int64_t)wg * (2 * kHeadDim) + h * kHeadDim + j], A);
    if (j == 0) {
        store_dev(&ws_ml[(int64_t)wg * 4 + h], M);
        store_dev(&ws_ml[(int64_t)wg * 4 + 2 + h], Ls);
    }
    stores_done_barrier();  // waves past thread 256 have exited: s_barrier counts live waves
    uint32_t* ctr = &counters[b * g.nkvh + kvh];
    if (tid == 0) s_last = (ticket_add(ctr) == (uint32_t)(nch - 1));
    __syncthreads();
    if (!s_last) return;

    // Last arrival: merge the nch partials of (b, kv head) in chunk order:
    // M = max of the chunk maxima, then sum_i 2^(m_i - M) * (l_i, acc_i).
    // Every chunk holds at least one real key, so every m_i is finite.  Each
    // thread requests the (m, l) of its head and its element of every chunk
    // of a batch of 32 at once, as plain device-coherent (sc1) loads: a batch
    // costs one memory round trip and the arithmetic has no branches.
    const int64_t it0 = P.wg_base[b] + kvh * nch;
    const __amdgpu_buffer_rsrc_t acc_res = make_rsrc(ws_acc + it0 * (2 * kHeadDim), nch * (2 * kHeadDim) * 4);
    const __amdgpu_buffer_rsrc_t ml_res = make_rsrc(ws_ml + it0 * 4, nch * 16);
    constexpr int kBatch = kDecodeMergeBatch;
    auto ld_ml = [&](int i, int k) {  // k: 0 = m, 2 = l
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ml_res, (i * 4 + k + h) * 4, 0, kSc1));
    };
    auto ld_acc = [&](int i) {
        return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                             acc_res, (i * (2 * kHeadDim) + h * kHeadDim + j) * 4, 0, kSc1));
    };
    float lsum = 0.0f, acc = 0.0f;
    // One round trip for N >= nch chunks (N a compile-time batch, so only
    // about as many loads are issued as there are chunks).
    auto merge_one_batch = [&](auto n_tag) {
        constexpr int N = decltype(n_tag)::value;
        float mv[N], lv[N], xv[N];
#pragma unroll
        for (int u = 0; u < N; ++u) {
            const int i = u < nch ? u : 0;
            mv[u] = ld_ml(i, 0);
            lv[u] = ld_ml(i, 2);
            xv[u] = ld_acc(i);
        }
        float M = mv[0];
#pragma unroll
        for (int u = 1; u < N; ++u) M = fmaxf(M, mv[u]);  // repeats of chunk 0 change nothing
#pragma unroll
        for (int u = 0; u < N; ++u) {
            const float wgt = u < nch ? fast_exp2(mv[u] - M) : 0.0f;
            lsum = fmaf(lv[u], wgt, lsum);
            acc = fmaf(xv[u], wgt, acc);
        }
    };
    if (nch <= 4) {
        merge_one_batch(std::integral_constant<int, 4>{});
    } else if (nch <= 8) {
        merge_one_batch(std::integral_constant<int, 8>{});
    } else if (nch <= 16) {
        merge_one_batch(std::integral_constant<int, 16>{});
    } else if (nch <= kBatch) {
        merge_one_batch(std::integral_constant<int, kBatch>{});
    } else {
        float M = kNegInf;
        for (int i0 = 0; i0 < nch; i0 += kBatch) {
            float mv[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) mv[u] = ld_ml(i0 + u < nch ? i0 + u : i0, 0);
#pragma unroll
            for (int u = 0; u < kBatch; ++u) M = fmaxf(M, mv[u]);
        }
        for (int i0 = 0; i0 < nch; i0 += kBatch) {
            float mv[kBatch], lv[kBatch], xv[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int i = i0 + u < nch ? i0 + u : i0;
                mv[u] = ld_ml(i, 0);
                lv[u] = ld_ml(i, 2);
                xv[u] = ld_acc(i);
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const float wgt = i0 + u < nch ? fast_exp2(mv[u] - M) : 0.0f;
                lsum = fmaf(lv[u], wgt, lsum);
                acc = fmaf(xv[u], wgt, acc);
            }
        }
    }
    ob[h * kHeadDim + j] = f2h(acc / lsum);
    if (tid == 0) ticket_reset(ctr);
}

template <bool FUSED>
hipError_t launch_w(int waves, const dim3& grid, hipStream_t stream, const CacheGeom& g,
                    int layer, const DecodePlan& P, const f16* qin, const f16* q_gain,
                    const f16* k_gain, const f16* cos_tab, const f16* sin_tab, f16* out,
                    const DecodeWs& ws) {
    switch (waves) {
        case 4:
            hipLaunchKernelGGL((decode_attn_kernel<FUSED, 4>), grid, dim3(4 * 64), 0, stream, g,
                               layer, P, qin, q_gain, k_gain, cos_tab, sin_tab, out, ws.acc,
                               ws.ml, ws.counters);
            break;
        case 8:
            hipLaunchKernelGGL((decode_attn_kernel<FUSED, 8>), grid, dim3(8 * 64), 0, stream, g,
                               layer, P, qin, q_gain, k_gain, cos_tab, sin_tab, out, ws.acc,
                               ws.ml, ws.counters);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_attn(bool fused, int waves, const CacheGeom& g, int layer,
                              const DecodePlan& P, int total_wgs, const f16* q_or_qkv,
                              const f16* q_gain, const f16* k_gain, const f16* cos_tab,
                              const f16* sin_tab, f16* out, const DecodeWs& ws,
                              hipStream_t stream) {
    if (total_wgs <= 0) return hipSuccess;
    if (total_wgs > ws.items) return hipErrorInvalidValue;
    const dim3 grid(total_wgs);
    if (fused)
        return launch_w<true>(waves, grid, stream, g, layer, P, q_or_qkv, q_gain, k_gain, cos_tab,
                              sin_tab, out, ws);
    return launch_w<false>(waves, grid, stream, g, layer, P, q_or_qkv, q_gain, k_gain, cos_tab,
                           sin_tab, out, ws);
}

}  // namespace qasr
