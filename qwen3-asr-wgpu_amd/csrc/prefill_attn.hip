// prefill_attn.hip -- stage (c): causal GQA prefill attention on fp16 MFMA
// (v_mfma_f32_32x32x16_f16, gfx950) with online softmax, for s rows at
// positions kv_start.. against cache rows 0..kv_start+s-1 (chunked prefill /
// KV-prefix reuse when kv_start > 0).
//
// Replaces the reference's repeat_kv -> prefill_gemm_causal -> softmax_causal
// -> prefill_gemm_causal_av pipeline and its slab variant (src/shaders.rs:
// 3058-4184, orchestrated in src/decoder.rs:4856-5098): no K/V expansion, no
// f16 score or probability matrix in memory.  Semantics: src/cpu_decoder.rs:
// 292-365 with rows = s, q0 = kv_start.
//
// Work item = (kv head, block of 64 query rows, split of the key range).
// 4 waves: wave w takes q head 2*kvh + (w&1) and rows (w>>1)*32..+32 of the
// block, so both q heads of a kv head share each K/V tile staged in LDS.
// Items are laid out kv-head minor (blockIdx % nkvh = kv head): with 8 kv
// heads and workgroups dealt round-robin to the 8 XCDs, every row block and
// split of one kv head runs on the same XCD and reuses its K/V through that
// XCD's L2.
// Each wave computes S^T = K Q^T (keys on the MFMA M axis, queries on N), so a
// lane owns one query column: row max / row sum need one cross-half shuffle,
// and the probabilities are already in the B-operand layout of O^T += V^T P^T.
// K/V tiles of 64 keys are double-buffered in LDS (V transposed to [dim][key],
// key columns XOR-swizzled per 8 dims, while it is stored): the next tile's global loads (buffer loads whose range
// ends at the row block's last key, so the tail reads zeros) are in flight
// while the current tile's MFMAs run, with one barrier per tile.  Only tiles
// that straddle the diagonal are masked, and O is rescaled only when a row
// max moved.
// When the key range of a row block is split, each item publishes its partial
// (max, sum, unnormalised O) with device-scope stores and the last to arrive
// merges (ticket), as in the decode kernel.

#include <algorithm>

#include "kernels.hpp"

namespace qasr {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = kPrefillWaves;
constexpr int kThreads = kWaves * 64;
// The split workspace holds exactly what one wave publishes: its 4 x 16
// accumulator registers for 64 lanes, and (m, l) for 64 lanes.
static_assert(kPrefillWaveFloats == 4 * 16 * 64, "partial O record size");
static_assert(kPrefillWaveMl == 2 * 64, "partial (m, l) record size");
constexpr int kRowsPerBlock = kPrefillRows;
constexpr int kTileKeys = 64;
constexpr int kKPad = kHeadDim + 8;   // Ks row stride (halves)
constexpr int kVPad = kTileKeys + 8;  // Vt row stride (halves)
constexpr int kKsHalves = kTileKeys * kKPad;
// One past the last V^T element (row 127 at skew 4*15, position 63; see
// vt_index), rounded up to 16 bytes so both buffers stay 16-byte aligned.
constexpr int kVtHalves = ((kHeadDim - 1) * kVPad + 4 * ((kHeadDim - 1) >> 3) + kTileKeys + 7) / 8 * 8;
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ float16v mfma32(const half8v& a, const half8v& b, const float16v& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Lanes l and l^32 hold the two key halves of one query column.  One
// v_permlane32_swap gives every lane both values (no LDS round trip).
__device__ __forceinline__ float halves_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}

// One 64-key tile of K and V: 4 + 4 dwordx4 per thread (thread t, chunk c
// covers key (c*256+t)/16, dims ((c*256+t)%16)*8..+8).
struct TileRegs {
    uint4 k[4];
    uint4 v[4];
};

__device__ __forceinline__ void load_tile(__amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr,
                                          int k0, int tid, TileRegs& t) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int off = (k0 * kHeadDim + (c * kThreads + tid) * 8) * 2;
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(kr, off, 0, 0);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(vr, off, 0, 0);
        t.k[c] = make_uint4(a.x, a.y, a.z, a.w);
        t.v[c] = make_uint4(b.x, b.y, b.z, b.w);
    }
}

// V^T element (dim, key) of a 64-key tile, in halves.
//  * Within each 16-key block, key bits 2 and 3 are swapped, so the keys one
//    lane feeds to a k-step, 4g + {0..3} and 4g + {8..11}, are 8 contiguous
//    halves (one ds_read2_b64 into the 4 registers of the operand).
//  * Row dim starts at dim*kVPad + 4*(dim/8): the 16 lanes that store dims
//    8j + e of one key then fall 2*j dwords apart, on 16 different banks.
//    The skew never decreases with dim and kVPad - 64 >= 4, so rows never
//    overlap.
__device__ __forceinline__ int vt_pos(int key) {
    return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}
__device__ __forceinline__ int vt_index(int dim, int key) {
    return dim * kVPad + 4 * (dim >> 3) + vt_pos(key);
}
static_assert(kVPad - kTileKeys >= 4, "V^T rows would overlap");

__device__ __forceinline__ void store_tile(const TileRegs& t, f16* Ks, f16* Vt, int tid) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int idx = c * kThreads + tid;
        const int key = idx >> 4, dseg = (idx & 15) * 8;
        *(uint4*)&Ks[key * kKPad + dseg] = t.k[c];
        H8 v;
        v.u = t.v[c];
#pragma unroll
        for (int e = 0; e < 8; ++e) Vt[vt_index(dseg + e, key)] = v.e[e];
    }
}

// Merge of the nsp split-K partials of one wave's 32 rows (lane = query row):
// returns the merged row sum and leaves the merged, unnormalised output in o.
// The partials are combined in index order whichever workgroup arrives last,
// so the result is bitwise reproducible.  Pass 1: the row max M (16 m values
// requested per memory round trip).  Pass 2: partials in groups of G, their
// (m, l) and, per 8-element chunk, the G x 8 accumulator values requested
// together.  Unused slots of a group read partial 0's record and drop it.
template <int G>
__device__ __forceinline__ float merge_partials(const float* mlw, const float* ow, int nsp,
                                                float16v (&o)[4]) {
    float M = kNegInf;
    for (int i0 = 0; i0 < nsp; i0 += 16) {
        float mm[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int i = i0 + u;
            const float v = load_dev(mlw + (int64_t)(i < nsp ? i : 0) * kPrefillItemMl);
            mm[u] = i < nsp ? v : kNegInf;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) M = fmaxf(M, mm[u]);
    }
    float Ls = 0.0f;
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = (float16v){};
    for (int i0 = 0; i0 < nsp; i0 += G) {
        float w[G];
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const int i = i0 + u;
            const float* rec = mlw + (int64_t)(i < nsp ? i : 0) * kPrefillItemMl;
            const float mi = load_dev(rec), li = load_dev(rec + 64);
            w[u] = (i >= nsp || mi == kNegInf) ? 0.0f : fast_exp2(mi - M);
            Ls = fmaf(i < nsp ? li : 0.0f, w[u], Ls);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {  // element chunk c: o[c/2][8*(c%2) .. +8]
            float x[G][8];
#pragma unroll
            for (int u = 0; u < G; ++u) {
                const int i = i0 + u;
                const float* src = ow + (int64_t)(i < nsp ? i : 0) * kPrefillItemFloats + c * 8 * 64;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float v = load_dev(src + e * 64);
                    x[u][e] = i < nsp ? v : 0.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < G; ++u)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    o[c >> 1][8 * (c & 1) + e] = fmaf(x[u][e], w[u], o[c >> 1][8 * (c & 1) + e]);
            __builtin_amdgcn_sched_barrier(0);  // keep the next chunk's loads after this one
        }
    }
    return Ls;
}

__global__ __launch_bounds__(kThreads, 2) void prefill_attn_kernel(
    PrefillArgs a, PrefillPlan P, float* __restrict__ ws_o, float* __restrict__ ws_ml,
    uint32_t* __restrict__ counters) {
    __shared__ __attribute__((aligned(16))) f16 Ks[2][kKsHalves];
    __shared__ __attribute__((aligned(16))) f16 Vt[2][kVtHalves];
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n = lane & 31;  // query column within the wave's 32 rows
    const int g = lane >> 5;  // k-slot group of the MFMA operands

    const int kvh = blockIdx.x % a.nkvh;
    const int rem = blockIdx.x / a.nkvh;
    const int item = kvh * P.items_per_kvh + rem;  // canonical index (workspace)
    int rb = 0;
    {
        int lo = 0, hi = P.nrb - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (P.sp_base[mid] <= rem) lo = mid; else hi = mid - 1;
        }
        rb = lo;
    }
    const int sp = rem - P.sp_base[rb];
    const int nsp = P.sp_base[rb + 1] - P.sp_base[rb];
    const int row0 = rb * kRowsPerBlock;
    const int kend = a.kv_start + min(row0 + kRowsPerBlock, a.s);  // keys < kend
    const int ntiles = (kend + kTileKeys - 1) / kTileKeys;
    const int t_begin = sp * P.tps;
    const int t_end = min(t_begin + P.tps, ntiles);

    const int hh = wave & 1;
    const int head = kvh * kRep + hh;
    const int wrow0 = row0 + (wave >> 1) * 32;  // first row of this wave
    const int r = wrow0 + n;                      // this lane's query row
    const bool row_ok = r < a.s;
    const int qpos = a.kv_start + r;
    const int ldq = a.nqh * kHeadDim;

    const __amdgpu_buffer_rsrc_t kres = make_rsrc(a.k + kvh * a.head_stride, kend * kHeadDim * 2);
    const __amdgpu_buffer_rsrc_t vres = make_rsrc(a.v + kvh * a.head_stride, kend * kHeadDim * 2);

    TileRegs pre;
    load_tile(kres, vres, t_begin * kTileKeys, tid, pre);

    // Q^T as B operand: k-step ks covers dims ks*16 + g*8 .. +8.
    half8v qb[8];
    {
        const f16* qrow = a.q + (int64_t)(row_ok ? r : 0) * ldq + head * kHeadDim + g * 8;
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            H8 t;
            t.u = row_ok ? *(const uint4*)(qrow + ks * 16) : make_uint4(0, 0, 0, 0);
            qb[ks] = t.h;
        }
    }

    float m = kNegInf, lsum = 0.0f;
    float16v o[4];
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = (float16v){};

    // V^T operand of k-step w4, dims db*32..+32: keys 16*w4 + 4*g + {0..3,
    // 8..11} of dim db*32 + n sit at vt_index(dim, 16*w4 + 4*g) .. +8, which
    // is the per-lane vlane plus a compile-time offset (dim>>3 = 4*db + n/8).
    const int vlane = n * kVPad + 4 * (n >> 3) + 8 * g;
    const half2v ones2 = {(f16)1.0f, (f16)1.0f};

    store_tile(pre, Ks[0], Vt[0], tid);
    __syncthreads();

    for (int t = t_begin; t < t_end; ++t) {
        const int buf = (t - t_begin) & 1;
        const int k0 = t * kTileKeys;
        if (t + 1 < t_end) load_tile(kres, vres, k0 + kTileKeys, tid, pre);
        const f16* ks_ = Ks[buf];
        const f16* vt_ = Vt[buf];

        // S^T: keys kb*32 + (8*(i/4) + 4*g + i%4) x query n, accumulated over dims.
        float16v st[2] = {(float16v){}, (float16v){}};
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const half8v ka = *(const half8v*)&ks_[(kb * 32 + n) * kKPad + ks * 16 + g * 8];
                st[kb] = mfma32(ka, qb[ks], st[kb]);
            }
        // Row max on the raw scores (the scale is positive), scaled once; the
        // scale is then folded into the exponent: p = 2^(s*scale_log2 - m).
        float mx = kNegInf;
        if (k0 + kTileKeys - 1 <= a.kv_start + wrow0) {  // whole tile visible to the wave
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) mx = fmaxf(mx, st[kb][i]);
        } else {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = k0 + kb * 32 + 8 * (i >> 2) + 4 * g + (i & 3);
                    const float v = key > qpos ? kNegInf : st[kb][i];
                    st[kb][i] = v;
                    mx = fmaxf(mx, v);
                }
        }
        mx = halves_max(mx) * a.scale_log2;
        const float mn = fmaxf(m, mx);
        const float mu = mn == kNegInf ? 0.0f : mn;
        const float alpha = fast_exp2(m - mu);
        m = mn;
        // P^T in the B-operand layout, k-step w4 covering tile keys
        // 16*w4 + 4*g + {0..3, 8..11}; its row sum is taken from the same f16
        // values the MFMA consumes (v_dot2 against ones, f32 accumulate).
        half8v pb[4];
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                pb[w4][j] = (f16)fast_exp2(fmaf(st[w4 >> 1][8 * (w4 & 1) + j], a.scale_log2, -mu));
        float ps = 0.0f;
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4)
#pragma unroll
            for (int q2 = 0; q2 < 4; ++q2) {
                const half2v pr = {pb[w4][2 * q2], pb[w4][2 * q2 + 1]};
                ps = __builtin_amdgcn_fdot2(pr, ones2, ps, false);
            }
        ps = halves_sum(ps);
        lsum = lsum * alpha + ps;
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int db = 0; db < 4; ++db) o[db] *= alpha;
        }

        // O^T += V^T P^T.
#pragma unroll
        for (int w4 = 0; w4 < 4; ++w4) {
#pragma unroll
            for (int db = 0; db < 4; ++db) {
                const f16* vp = vt_ + vlane + db * (32 * kVPad + 16) + 16 * w4;
                const half4v lo = *(const half4v*)vp;
                const half4v hi = *(const half4v*)(vp + 4);
                const half8v va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
                o[db] = mfma32(va, pb[w4], o[db]);
            }
        }
        if (t + 1 < t_end) store_tile(pre, Ks[buf ^ 1], Vt[buf ^ 1], tid);
        __syncthreads();
    }

    // o[db][i] holds dim db*32 + 8*(i/4) + 4*g + i%4 of query row r.
    f16* orow = a.out + (int64_t)r * ldq + head * kHeadDim;
    if (nsp == 1) {
        if (row_ok) {
            const float inv = 1.0f / lsum;
#pragma unroll
            for (int db = 0; db < 4; ++db) {
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    half4v h4;
#pragma unroll
                    for (int e = 0; e < 4; ++e) h4[e] = (f16)(o[db][q4 * 4 + e] * inv);
                    *(half4v*)(orow + db * 32 + 8 * q4 + 4 * g) = h4;
                }
            }
        }
        return;
    }

    // Partial of this wave: 64 accumulator elements x 64 lanes, element-major
    // (element e of lane l at [e][l]) so every store and load instruction
    // moves 256 contiguous bytes; then (m, l) per lane.  Published with
    // device-scope stores (see stores_done_barrier).
    float* po = ws_o + (int64_t)item * kPrefillItemFloats + wave * kPrefillWaveFloats;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) store_dev(po + (db * 16 + i) * 64 + lane, o[db][i]);
    float* pml = ws_ml + (int64_t)item * kPrefillItemMl + wave * kPrefillWaveMl;
    store_dev(pml + lane, m);
    store_dev(pml + 64 + lane, lsum);
    stores_done_barrier();
    uint32_t* ctr = &counters[kvh * P.nrb + rb];
    if (tid == 0) s_last = (ticket_add(ctr) == (uint32_t)(nsp - 1));
    __syncthreads();
    if (!s_last) return;

    // Last arrival: merge the nsp partials of this (kv head, row block); each
    // wave merges its own 32 rows.
    const int it0 = kvh * P.items_per_kvh + P.sp_base[rb];
    const float* mlw = ws_ml + (int64_t)it0 * kPrefillItemMl + wave * kPrefillWaveMl + lane;
    const float* ow = ws_o + (int64_t)it0 * kPrefillItemFloats + wave * kPrefillWaveFloats + lane;
    float Ls;
    if (nsp <= 2)
        Ls = merge_partials<2>(mlw, ow, nsp, o);
    else
        Ls = merge_partials<8>(mlw, ow, nsp, o);
    if (row_ok) {
        const float inv = 1.0f / Ls;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                half4v h4;
#pragma unroll
                for (int e = 0; e < 4; ++e) h4[e] = (f16)(o[db][q4 * 4 + e] * inv);
                *(half4v*)(orow + db * 32 + 8 * q4 + 4 * g) = h4;
            }
    }
    if (tid == 0) ticket_reset(ctr);
}

}  // namespace

PrefillPlan plan_prefill(int s, int kv_start, int nkvh, int tiles_per_split) {
    PrefillPlan P{};
    P.nrb = (s + kRowsPerBlock - 1) / kRowsPerBlock;
    P.tps = tiles_per_split;
    P.sp_base[0] = 0;
    for (int rb = 0; rb < P.nrb; ++rb) {
        const int kend = kv_start + std::min((rb + 1) * kRowsPerBlock, s);
        const int ntiles = (kend + kTileKeys - 1) / kTileKeys;
        P.sp_base[rb + 1] = P.sp_base[rb] + (ntiles + P.tps - 1) / P.tps;
    }
    P.items_per_kvh = P.sp_base[P.nrb];
    (void)nkvh;
    return P;
}

hipError_t launch_prefill_attn(const PrefillArgs& a, const PrefillPlan& P, const PrefillWs& ws,
                               hipStream_t stream) {
    const int items = P.items_per_kvh * a.nkvh;
    if (items <= 0) return hipSuccess;
    if (items > ws.items || P.nrb > kMaxRowBlocks) return hipErrorInvalidValue;
    hipLaunchKernelGGL(prefill_attn_kernel, dim3(items), dim3(kThreads), 0, stream, a, P, ws.o,
                       ws.ml, ws.counters);
    return hipGetLastError();
}

}  // namespace qasr
