// decode_attn.hip -- stage (b): GQA decode attention over ragged per-slot
// contexts, split-K with an in-kernel merge; optionally fused with stage (a).
//
// Replaces the reference's gqa_decode_single[_slots], gqa_decode_split_p1_pair
// and gqa_split_merge (src/shaders.rs:1881-2905, planned in src/decoder.rs:
// 1932-2025 and 3348-3451).  Semantics: src/cpu_decoder.rs:292-365 with one
// query row, i.e. softmax(q.k_t * scale) . v over keys t < cur_len.
//
// Granules and runs.  An entry's keys are cut into granules whose size is a
// function of the entry's own length only (the host's plan: a multiple of 256
// keys, at most kDecodeMaxGranules of them).  Each granule yields one partial
// (max, sum, unnormalised output per q head), and the partials of an entry
// are merged in granule order.  So the bits of an entry's output depend on
// its length and its keys, never on its batch mates: the reference's
// `--batch N` output is byte-identical to `--batch 1` (src/decoder.rs:
// 1930-1931, README "byte-identical"), and so is this kernel's.  What the
// batch changes is only which workgroup runs which granules: a workgroup
// takes a run of consecutive granules of one (entry, kv head), so the host
// can spread any batch over about one workgroup per CU.
//
// Work decomposition (one launch for the whole batch):
//   workgroup = (batch entry b, run of granules, kv head), 4 waves.
//   Both q heads of the kv head (GQA 2:1) are computed from one K/V read.
//   A workgroup pass covers 128 contiguous keys, wave w taking keys 32w..+32:
//   8 dwordx4 buffer loads of K and 8 of V per lane, each instruction
//   reading 1 KiB contiguous (4 keys x 256 B, lane l -> key l/16, dims
//   (l%16)*8..+8), so every instruction is fully coalesced.  The buffer
//   resources end at the run's last key, so the hardware range check returns
//   zeros past it (those scores are masked).
//   q.k: v_dot2_f32_f16 on the lane's 8 dims, then a transposing 16-lane DPP
//   reduction that leaves each lane with one (key, head) score.  Softmax is
//   online per (16-lane row, head) in the exp2 domain; the row's 16
//   probabilities reach the V layout through LDS and P.V accumulates in f32
//   (v_fma_mix on packed f16).  At each granule's end each wave merges its
//   4 rows through lane swaps (no LDS round trip, no workgroup barrier: the
//   waves stream independently) into its wave partial, kept in LDS, and the
//   rows start over.  After the run the 4 wave partials of each granule
//   combine, in wave order, into the granule's partial: an entry with one
//   granule writes its output; a (entry, kv head) whose granules all ran in
//   this workgroup merges them there; otherwise the run's partials are
//   published with device-scope stores and the last workgroup to arrive
//   (ticket) merges all of them, issuing its loads at once: no second launch
//   and no L2-wide cache maintenance.  Both merges combine the same values in
//   the same order.
//
// Fused variant (stage (a) + (b)): the workgroup recomputes its two q heads
// from the raw qkv row (bit-identical to the stage-(a) kernel); the workgroup
// owning the last granule also ropes the new K row, appends K and V to the
// cache and substitutes them for the cache load of that key.  The first K/V
// pass is requested before the workgroup waits for its query inputs, so the
// prologue runs under that pass's latency.

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
constexpr int W = kDecodeWaves;
constexpr int kWgKeys = W * kDecodeTileKeys;  // keys per workgroup pass
static_assert(2 * kWgKeys == kDecodeGranuleQuantum, "a granule is an even number of workgroup passes");
constexpr int kMaxG = kDecodeMaxGranules;
constexpr int kMaxRunG = kDecodeMaxRunGranules;

// Lane swaps between rows (16-lane groups): pair_rows gives every lane the
// value of the even (first) and odd (second) row of its row pair, halves the
// value of the lower (first) and upper (second) 32 lanes, at the lane's
// position in the row / half.
__device__ __forceinline__ void pair_rows(float v, float& even, float& odd) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    even = __uint_as_float(r[0]);
    odd = __uint_as_float(r[1]);
}
__device__ __forceinline__ void halves(float v, float& lo, float& hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    lo = __uint_as_float(r[0]);
    hi = __uint_as_float(r[1]);
}

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

template <bool FUSED>
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
    __shared__ float s_inv[3];
    __shared__ __attribute__((aligned(16))) float s_sq[3][kHeadDim];  // f32 squares of q0, q1, k
    __shared__ float s_p[W][64];
    // Wave partials of the run's granules: (max, sum) per head and the
    // unnormalised output of both heads.
    __shared__ float s_wm[kMaxRunG][W][2];
    __shared__ float s_wl[kMaxRunG][W][2];
    // The run's wave partials (unnormalised output of both heads), and once
    // they are published, the last arrival's copies of the pair's granule
    // outputs: one buffer.
    __shared__ __attribute__((aligned(16))) float s_big[kMaxG * 2 * kHeadDim];
    static_assert(kMaxRunG * W <= kMaxG, "the wave partials fit the merge buffer");
    float(*s_wa)[W][2][kHeadDim] = reinterpret_cast<float(*)[W][2][kHeadDim]>(s_big);
    float(*s_x)[2 * kHeadDim] = reinterpret_cast<float(*)[2 * kHeadDim]>(s_big);
    __shared__ int s_last;
    // The last arrival's copies of the granule partials: (m0, m1, l0, l1)
    // and the unnormalised output of both heads per granule.
    __shared__ __attribute__((aligned(16))) float s_ml[kMaxG][4];

    const int wg = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int row = lane >> 4;  // key within a 4-key load
    const int seg = lane & 15;  // 8-dim segment

    // Entry of this workgroup = number of later entry starts at or before it:
    // lane i tests wg_base[i + 1], one load per lane and a ballot, no search.
    // Lane i reads every plan field of entry i in that same round trip (the
    // argument arrays hold kMaxBatch = 64 entries, so every read is in
    // bounds, and unconditional, so no branch holds back the other argument
    // loads); entry b's fields are then lane reads, not a second dependent
    // load before the first K/V request.
    static_assert(kMaxBatch == 64, "one lane per entry");
    const int e_len = P.len[lane], e_gran = P.gran[lane], e_run = P.run[lane];
    const int e_slot = P.slot[lane], e_wg0 = P.wg_base[lane], e_wg1 = P.wg_base[lane + 1];
    const int e_part = P.part_base[lane];
    const int b = __popcll(__ballot(lane + 1 < P.batch && e_wg1 <= wg));
    const int L = __builtin_amdgcn_readlane(e_len, b);
    const int G = __builtin_amdgcn_readlane(e_gran, b);
    const int run = __builtin_amdgcn_readlane(e_run, b);
    const int ngr = (L + G - 1) / G;        // granules of the entry (per kv head)
    const int nw = (ngr + run - 1) / run;   // workgroups per kv head
    // kv head minor: workgroup i runs on XCD i mod 8, so with 8 kv heads every
    // XCD gets one run of each size.  Runs end at the entry's end: the last
    // holds the (possibly short) last granule, the first any remainder.
    const int rel = wg - __builtin_amdgcn_readlane(e_wg0, b);
    const int kvh = rel % g.nkvh;
    const int r = rel / g.nkvh;
    const int g1 = ngr - (nw - 1 - r) * run;
    const int g0 = max(0, g1 - run);
    const int key0 = g0 * G;
    const int key1 = min(g1 * G, L);
    const int nkeys = key1 - key0;
    const int ppg = G / kWgKeys;                    // passes per granule
    const int npass = (nkeys + 2 * kWgKeys - 1) / (2 * kWgKeys) * 2;  // even
    const int nqh = P.nqh;
    const int h0 = kvh * kRep;
    f16* Kc = g.base + __builtin_amdgcn_readlane(e_slot, b) * g.slot_stride + layer * g.layer_stride +
              kvh * g.head_stride;
    f16* Vc = Kc + g.kv_stride;
    // Resources start at the run's first key and end at its last.
    const int rbytes = nkeys * (kHeadDim * 2);
    const __amdgpu_buffer_rsrc_t kres = make_rsrc(Kc + (int64_t)key0 * kHeadDim, rbytes);
    const __amdgpu_buffer_rsrc_t vres = make_rsrc(Vc + (int64_t)key0 * kHeadDim, rbytes);
    const int tw = wave * kDecodeTileKeys;  // this wave's first key in a pass

    // The query inputs (the raw qkv heads and the gain / cos / sin rows, or q
    // itself) come in by direct global -> LDS copies, requested first; the
    // first K/V pass is requested right after them, and only then does the
    // workgroup wait for the copies (by count: they are older than the pass),
    // so the K/V stream starts without waiting for a round trip and the
    // prologue runs while the first pass is in flight.  The passes are issued
    // in order (scheduling barriers): the loop waits for the older pass by
    // count while the newer one stays in flight.
    const int pos = L - 1;
    const bool owner = FUSED && (r == nw - 1);
    // The query-input pointers are kernel arguments too: held in scalar
    // registers here, their loads join the plan's round trip above instead
    // of a round trip of their own inside the copy branches below (which the
    // K/V requests follow).
    if constexpr (FUSED)
        asm volatile("" ::"s"(qin), "s"(q_gain), "s"(k_gain), "s"(cos_tab), "s"(sin_tab));
    else
        asm volatile("" ::"s"(qin));
    if constexpr (FUSED) {
        const int64_t tot = (int64_t)(nqh + 2 * g.nkvh) * kHeadDim;
        const f16* qkv_row = qin + b * tot;
        if (wave == 0) {  // lane l: head l/16 (q0, q1, k, v), 16-byte piece l%16
            const int which = lane >> 4;
            const int hoff = which < 2 ? (h0 + which) : which == 2 ? (nqh + kvh) : (nqh + g.nkvh + kvh);
            dma16(make_rsrc_words(qkv_row, (int)(tot * 2)), hoff * (kHeadDim * 2) + seg * 16,
                  lds_addr(&s_raw[0][0]));
        } else if (wave == 1 && lane < 16) {
            dma16(make_rsrc_words(q_gain, kHeadDim * 2), seg * 16, lds_addr(&s_tab[0][0]));
            dma16(make_rsrc_words(k_gain, kHeadDim * 2), seg * 16, lds_addr(&s_tab[1][0]));
            dma16(make_rsrc_words(cos_tab + (int64_t)pos * kHeadDim, kHeadDim * 2), seg * 16,
                  lds_addr(&s_tab[2][0]));
            dma16(make_rsrc_words(sin_tab + (int64_t)pos * kHeadDim, kHeadDim * 2), seg * 16,
                  lds_addr(&s_tab[3][0]));
        }
    } else if (wave == 0 && lane < 32) {  // lane l: q head l/16, 16-byte piece l%16
        const f16* qb = qin + (int64_t)b * nqh * kHeadDim + h0 * kHeadDim;
        dma16(make_rsrc_words(qb, 2 * kHeadDim * 2), lane * 16, lds_addr(&s_q[0][0]));
    }

    H8 ka[8], va[8], kb[8], vb[8];
    load_pass(kres, tw, row, seg, ka);
    load_pass(vres, tw, row, seg, va);
    __builtin_amdgcn_sched_barrier(0);
    // This wave's copies are older than the 16 pass loads just issued.
    __builtin_amdgcn_s_waitcnt(0x4F70);  // vmcnt(16)
    __syncthreads();

    H8 q0, q1;
    if constexpr (FUSED) {
        // The squares (exact in f32) come from every thread at once; the
        // serial path is then the reference's 128 dependent adds alone.
        static_assert(W * 64 == 2 * kHeadDim, "one thread per q element");
        {
#pragma clang fp contract(off)
            const float x = h2f(s_raw[tid >> 7][tid & 127]);
            s_sq[tid >> 7][tid & 127] = x * x;
            if (owner && tid < kHeadDim) {
                const float xk = h2f(s_raw[2][tid]);
                s_sq[2][tid] = xk * xk;
            }
        }
        __syncthreads();
        if (tid < 3 && (tid < 2 || owner)) s_inv[tid] = head_inv_rms_squares_all(s_sq[tid], P.eps);
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
    }
    q0 = s_q[0][seg];
    q1 = s_q[1][seg];

    __builtin_amdgcn_sched_barrier(0);
    load_pass(kres, tw + kWgKeys, row, seg, kb);
    load_pass(vres, tw + kWgKeys, row, seg, vb);
    __builtin_amdgcn_sched_barrier(0);

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
    const int new_rel = pos - key0;  // the appended key, relative to the run (owner only)

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

    // One thread per (head, dim): h, j.  Partial records of this (entry, kv
    // head): part0 + granule.
    const int h = tid >> 7, j = tid & 127;
    f16* ob = out + (int64_t)b * nqh * kHeadDim + h0 * kHeadDim;
    const int64_t part0 = (int64_t)__builtin_amdgcn_readlane(e_part, b) + (int64_t)kvh * ngr;

    // Partial merge a <- a (+) b of two row states (each lane: (m, l) of the
    // head of its parity, 8 dims of both heads): M = max, then each side
    // weighted by 2^(m - M) (0 for a side without keys).  The other head's
    // weights come from the neighbouring lane.
    auto combine = [&](float& m, float& l, float (&x0)[8], float (&x1)[8], float mb, float lb,
                       const float (&y0)[8], const float (&y1)[8]) {
        const float M = fmaxf(m, mb);
        const float fa = m == kNegInf ? 0.0f : fast_exp2(m - M);
        const float fb = mb == kNegInf ? 0.0f : fast_exp2(mb - M);
        l = fmaf(lb, fb, l * fa);
        m = M;
        const float fax = dpp<kDppXor1>(fa), fbx = dpp<kDppXor1>(fb);
        const float fa0 = odd ? fax : fa, fb0 = odd ? fbx : fb;
        const float fa1 = odd ? fa : fax, fb1 = odd ? fb : fbx;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            x0[d] = fmaf(y0[d], fb0, x0[d] * fa0);
            x1[d] = fmaf(y1[d], fb1, x1[d] * fa1);
        }
    };

    // End of granule gi (relative to the run), per wave and without waiting
    // for the other waves: the wave's 4 rows merge as (row 0 (+) row 1) (+)
    // (row 2 (+) row 3) through lane swaps, and row 0's lanes leave the wave's
    // partial in LDS; then the rows start over.
    auto finalize = [&](int gi) {
        float m, l, x0[8], x1[8], mb, lb, y0[8], y1[8];
        pair_rows(m_run, m, mb);
        pair_rows(l_run, l, lb);
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            pair_rows(a0[d], x0[d], y0[d]);
            pair_rows(a1[d], x1[d], y1[d]);
        }
        combine(m, l, x0, x1, mb, lb, y0, y1);
        float n0, n1;
        halves(m, n0, n1);
        m = n0;
        mb = n1;
        halves(l, n0, n1);
        l = n0;
        lb = n1;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            halves(x0[d], n0, n1);
            x0[d] = n0;
            y0[d] = n1;
            halves(x1[d], n0, n1);
            x1[d] = n0;
            y1[d] = n1;
        }
        combine(m, l, x0, x1, mb, lb, y0, y1);
        if (lane < 16) {
            float* w0 = &s_wa[gi][wave][0][seg * 8];
            float* w1 = &s_wa[gi][wave][1][seg * 8];
            *(float4*)w0 = make_float4(x0[0], x0[1], x0[2], x0[3]);
            *(float4*)(w0 + 4) = make_float4(x0[4], x0[5], x0[6], x0[7]);
            *(float4*)w1 = make_float4(x1[0], x1[1], x1[2], x1[3]);
            *(float4*)(w1 + 4) = make_float4(x1[4], x1[5], x1[6], x1[7]);
            if (lane < 2) {  // lane 0: head 0's (m, l), lane 1: head 1's
                s_wm[gi][wave][lane] = m;
                s_wl[gi][wave][lane] = l;
            }
        }
        m_run = kNegInf;
        l_run = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) a0[d] = a1[d] = 0.0f;
    };

    // Workgroup passes p = 0, 1, ..: wave keys 128 p + tw .. +32, two per
    // iteration (a granule is an even number of passes, and an odd last pass
    // is followed by an empty one).  Every wave processes every pass: keys
    // past the run are masked, which leaves a row's state exactly as it was.
    // Only an entry's last granule can end inside a pass, and it is always
    // the last of its run.  The loop has one path and no workgroup barrier,
    // so the compiler keeps the next pass's loads in flight while the current
    // one is computed and the waves stream independently.
    for (int p = 0; p < npass; p += 2) {
        const int t0 = p * kWgKeys + tw;
        process(ka, va, t0);
        __builtin_amdgcn_sched_barrier(0);
        load_pass(kres, t0 + 2 * kWgKeys, row, seg, ka);
        load_pass(vres, t0 + 2 * kWgKeys, row, seg, va);
        process(kb, vb, t0 + kWgKeys);
        __builtin_amdgcn_sched_barrier(0);
        load_pass(kres, t0 + 3 * kWgKeys, row, seg, kb);
        load_pass(vres, t0 + 3 * kWgKeys, row, seg, vb);
        if ((p + 2) % ppg == 0 || p + 2 >= npass) finalize(p / ppg);
    }
    const int mine = g1 - g0;  // granules of this run
    __syncthreads();

    // Granule gi's partial (M, sum, unnormalised output of head h, dim j):
    // its 4 wave partials in wave order, each weighted by 2^(m_w - M).
    auto granule = [&](int gi, float& M, float& Lg, float& Ag) {
        float mw[W];
#pragma unroll
        for (int w = 0; w < W; ++w) mw[w] = s_wm[gi][w][h];
        M = mw[0];
#pragma unroll
        for (int w = 1; w < W; ++w) M = fmaxf(M, mw[w]);
        Lg = 0.0f;
        Ag = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float f = mw[w] == kNegInf ? 0.0f : fast_exp2(mw[w] - M);
            Lg = fmaf(s_wl[gi][w][h], f, Lg);
            Ag = fmaf(s_wa[gi][w][h][j], f, Ag);
        }
    };
    if (ngr == 1) {
        float M, Lg, Ag;
        granule(0, M, Lg, Ag);
        ob[h * kHeadDim + j] = f2h(Ag / Lg);
        return;
    }

    // Merge of the ngr granule partials in granule order: M = max of the
    // granule maxima, then sum_i 2^(m_i - M) * (l_i, acc_i).  Every granule
    // holds at least one real key, so every m_i is finite.  The LDS and the
    // workspace paths below do the same arithmetic on the same values in the
    // same order.
    if (nw == 1) {
        float M = kNegInf;
        for (int i = 0; i < ngr; ++i) {
            float mi, li, ai;
            granule(i, mi, li, ai);
            M = i == 0 ? mi : fmaxf(M, mi);
        }
        float lsum = 0.0f, acc = 0.0f;
        for (int i = 0; i < ngr; ++i) {
            float mi, li, ai;
            granule(i, mi, li, ai);
            const float wgt = fast_exp2(mi - M);
            lsum = fmaf(li, wgt, lsum);
            acc = fmaf(ai, wgt, acc);
        }
        ob[h * kHeadDim + j] = f2h(acc / lsum);
        return;
    }

    // Publish this run's partials (device-scope stores), four granules'
    // LDS reads at a time, then the ticket.
    for (int g4 = 0; g4 < mine; g4 += 4) {
        float mi[4], li[4], ai[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) granule(min(g4 + u, mine - 1), mi[u], li[u], ai[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (g4 + u < mine) {
                const int64_t it = part0 + g0 + g4 + u;
                store_dev(&ws_acc[it * (2 * kHeadDim) + h * kHeadDim + j], ai[u]);
                if (j == 0) {
                    store_dev(&ws_ml[it * 4 + h], mi[u]);
                    store_dev(&ws_ml[it * 4 + 2 + h], li[u]);
                }
            }
        }
    }
    stores_done_barrier();
    uint32_t* ctr = &counters[b * g.nkvh + kvh];
    if (tid == 0) s_last = (ticket_add_n(ctr, (uint32_t)mine) + (uint32_t)mine == (uint32_t)ngr);
    __syncthreads();
    if (!s_last) return;

    // Last arrival: each granule's partial (its 1 KiB output record and its
    // 16-byte (m0, m1, l0, l1) record) is copied into LDS by one wave, with
    // device-coherent (sc1) direct global -> LDS loads, all requested at
    // once: one memory round trip.  Then M = max of the granule maxima and
    // the weighted sums in granule order, the same arithmetic on the same
    // values as the in-workgroup merge.  (A plain loop: this code runs once
    // per pair, from a cold instruction cache.)
    {
        const u32x4v acc_res = make_rsrc_words(ws_acc + part0 * (2 * kHeadDim), ngr * (2 * kHeadDim) * 4);
        const u32x4v ml_res = make_rsrc_words(ws_ml + part0 * 4, ngr * 16);
        for (int u = wave; u < ngr; u += W) {
            dma16_sc1(acc_res, u * (2 * kHeadDim * 4) + lane * 16, lds_addr(&s_x[u][0]));
            if (lane == 0) dma16_sc1(ml_res, u * 16, lds_addr(&s_ml[u][0]));
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's copies landed
        __syncthreads();
    }
    float M = s_ml[0][h];
    for (int u = 1; u < ngr; ++u) M = fmaxf(M, s_ml[u][h]);
    float lsum = 0.0f, acc = 0.0f;
    for (int u = 0; u < ngr; ++u) {
        const float wgt = fast_exp2(s_ml[u][h] - M);
        lsum = fmaf(s_ml[u][2 + h], wgt, lsum);
        acc = fmaf(s_x[u][h * kHeadDim + j], wgt, acc);
    }
    ob[h * kHeadDim + j] = f2h(acc / lsum);
    if (tid == 0) ticket_reset(ctr);
}

}  // namespace

hipError_t launch_decode_attn(bool fused, const CacheGeom& g, int layer, const DecodePlan& P,
                              int total_wgs, const f16* q_or_qkv, const f16* q_gain,
                              const f16* k_gain, const f16* cos_tab, const f16* sin_tab, f16* out,
                              const DecodeWs& ws, hipStream_t stream) {
    if (total_wgs <= 0) return hipSuccess;
    if (P.part_base[P.batch] > ws.items) return hipErrorInvalidValue;
    const dim3 grid(total_wgs), block(W * 64);
    if (fused)
        hipLaunchKernelGGL((decode_attn_kernel<true>), grid, block, 0, stream, g, layer, P,
                           q_or_qkv, q_gain, k_gain, cos_tab, sin_tab, out, ws.acc, ws.ml,
                           ws.counters);
    else
        hipLaunchKernelGGL((decode_attn_kernel<false>), grid, block, 0, stream, g, layer, P,
                           q_or_qkv, q_gain, k_gain, cos_tab, sin_tab, out, ws.acc, ws.ml,
                           ws.counters);
    return hipGetLastError();
}

}  // namespace qasr
