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
// Work item = (kv head, block of 64 query rows, split of the key range), one
// 8-wave workgroup per CU (two waves per SIMD).  Row wave rw = wave & 3 takes
// q head 2*kvh + (rw&1) and rows (rw>>1)*32..+32 of the block, so both q
// heads of a kv head share each K/V tile in LDS; key group kg = wave >> 2
// takes keys 64*kg..+64 of every 128-key tile, and the two key groups of a
// row wave are merged through LDS at the end.  Two waves per SIMD let one
// wave's softmax (VALU) run while the other's MFMAs do.  Items are laid out
// kv-head minor (blockIdx % nkvh = kv head): with 8 kv heads and workgroups
// dealt round-robin to the 8 XCDs, every row block and split of one kv head
// runs on the same XCD and reuses its K/V through that XCD's L2.
//
// Each wave computes S^T = K Q^T (keys on the MFMA M axis, queries on N), so a
// lane owns one query column: row max / row sum need one cross-half swap,
// and the probabilities are already in the B-operand layout of O^T += V^T P^T.
// The running max is moved (and O rescaled) only when a row max exceeds it by
// more than 2^8, so p <= 256 and the rescale branch is rarely taken; the
// result is the same softmax.  Only key halves that straddle the diagonal are
// masked, and halves wholly past it are skipped.
// K/V tiles and the Q block are copied global -> LDS directly (buffer_load ...
// lds, rows past the last key or query clamped to it), the K/V tiles double
// buffered: the first two tiles and Q are requested together at the start,
// and the copy of tile t+2 goes into tile t's buffers as soon as every wave is
// done with them, so one tile is always in flight while another is consumed.
// In 16-row blocks of more than 4 tiles each wave copies only the keys it
// reads and waits for its own copies, so the loop has no barrier and two
// tiles can be in flight.
// Every copy is inline asm waited for by count, so nothing the compiler
// inserts waits for a copy issued later.
// When the key range of a row block is split, each item publishes its partial
// (max, sum, unnormalised O) with device-scope stores and the last to arrive
// merges (ticket), as in the decode kernel.

#include <algorithm>

#include "kernels.hpp"

namespace qasr {

namespace {

constexpr int kWaves = kPrefillWaves;            // row waves
constexpr int kAllWaves = kWaves * kPrefillKeyGroups;
constexpr int kThreads = kAllWaves * 64;
// The split workspace holds exactly what one wave publishes: its 4 x 16
// accumulator registers for 64 lanes, and (m, l) for 64 lanes.
static_assert(kPrefillWaveFloats == 4 * 16 * 64, "partial O record size");
static_assert(kPrefillWaveMl == 2 * 64, "partial (m, l) record size");
constexpr int kRowsPerBlock = kPrefillRows;
constexpr int kTileKeys = kPrefillTileKeys;         // keys per LDS tile
constexpr int kGroupKeys = kTileKeys / kPrefillKeyGroups;  // keys per key group
static_assert(kGroupKeys == 64, "a key group's half tile is one 64-key wave step");
constexpr int kTileHalves = kTileKeys * kHeadDim;  // one 32 KB K or V tile
constexpr float kNegInf = -__builtin_inff();
constexpr float kRescaleSlack = 8.0f;  // log2 of the largest p before the max moves

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) short4v lds_short4v;

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

// ---- LDS tile layouts ----------------------------------------------------
// LDS serves 16 lanes of a 16-byte read (or 32 lanes of an 8-byte read) per
// cycle from 64 banks, so each such lane group must cover 256 distinct bytes
// modulo 256.
//
// K tile: row r (key) is 256 contiguous bytes; its 16-byte chunk c (dims
// 8c..8c+7) sits at slot c ^ swz16(r).  swz16 permutes 0..15 over every 16
// consecutive rows, so the K operand read (16 consecutive rows, one chunk)
// hits 16 different slots.
__device__ __forceinline__ int swz16(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
// V tile: four slabs of 32 dims, [dims/32][row][32 dims], 8 KB each.  The
// transposing read of 4 consecutive rows x 32 dims is then 256 contiguous
// bytes, and every operand address is a per-lane base plus a constant.
//
// Both tiles arrive by direct global -> LDS copies of one KB per wave
// instruction, lane l at +16 l.  With NW waves (8, or 4 for 16-row blocks):
//   K: instruction j of wave w writes KB NW j + w: rows 4 (NW j + w) + l/16,
//      slot l%16 = chunk (l%16) ^ swz16(4w + l/16) (swz16 has period 16);
//   V: slab j (32 dims, 8 KB of 16-row KBs), row group w + NW i: KB
//      8j + w + NW i, rows 16 (w + NW i) + l/4, dims 32j + 8(l%4) .. +8.
// Per thread the global source row is fixed within the tile (plus 4 NW j for
// K; V instruction j reads the next 64 bytes of the same row).
// The copies are issued as inline asm (M0 = LDS destination): the compiler
// then does not wait for them before unrelated LDS reads of the other
// buffers; the kernel waits for them itself (vmcnt(0)) before each barrier.
// (make_rsrc_words, lds_addr and dma16 are in common.hpp.)
// Rows past the last key of the row block (only in its last tile) are read
// from row kend-1 instead: masked keys get p = 0, and 0 * (finite V) = 0,
// whereas an out-of-range copy would leave whatever the LDS held before.
// t0: first key of the tile; krow/vrow, kchunk/vchunk: this thread's row
// within the tile and byte offset within the row (see the layout above).
template <int NW>
__device__ __forceinline__ void dma_tile(u32x4v kr, u32x4v vr, int t0, int kend, int krow,
                                         int kchunk, int vrow, int vchunk, const f16* kdst,
                                         const f16* vdst, int wave) {
    static_assert((NW == 8 || NW == 4) && kTileKeys == 128, "copy pattern: 32 + 32 one-KB blocks per tile");
    const int last = kend - 1;
#pragma unroll
    for (int j = 0; j < 32 / NW; ++j) {
        const int rk = min(t0 + krow + 4 * NW * j, last);
        dma16(kr, rk * 256 + kchunk, lds_addr(kdst + (NW * j + wave) * 512));
    }
#pragma unroll
    for (int i = 0; i < 8 / NW; ++i) {
        const int rv = min(t0 + vrow + 16 * NW * i, last);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            dma16(vr, rv * 256 + vchunk + j * 64, lds_addr(vdst + (8 * j + wave + NW * i) * 512));
    }
}
// Copy instructions per thread and tile.
template <int NW>
constexpr int kTileCopies = 32 / NW + 4 * (8 / NW);

// The same tile layout copied by 16-row blocks (four waves, key group =
// wave): wave w copies exactly the 32 keys it reads, K rows 32w .. +31 (KBs
// 8w + j, rows 32w + 4j + l/16) and V rows 32w .. +31 of every slab (KB
// 8j + 2w + i, rows 32w + 16i + l/4), 16 instructions like dma_tile<4>.  A
// wave then waits for its own copies only (vmcnt), with no workgroup
// barrier, and keeps two tiles in flight.
__device__ __forceinline__ void dma_slice(u32x4v kr, u32x4v vr, int t0, int kend, const f16* kdst,
                                          const f16* vdst, int wave, int lane) {
    const int last = kend - 1;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int row = 32 * wave + 4 * j + (lane >> 4);
        dma16(kr, min(t0 + row, last) * 256 + ((lane & 15) ^ swz16(row)) * 16,
              lds_addr(kdst + (8 * wave + j) * 512));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int rv = min(t0 + 32 * wave + 16 * i + (lane >> 2), last);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            dma16(vr, rv * 256 + (lane & 3) * 16 + j * 64, lds_addr(vdst + (8 * j + 2 * wave + i) * 512));
    }
}

// Q block: 64 rows x the kv head's 2 q heads (512 contiguous bytes per row),
// copied like the tiles (instruction j of wave w of NW: LDS KB NW j + w, lane
// l at +16 l, i.e. row 2(NW j + w) + l/32, slot l%32).  Slot c of row r holds
// 16-byte chunk c ^ (r & 15), so the operand read (16 consecutive rows, one
// chunk each) hits 16 different slots.  Rows past the block's last row are
// read from row s-1 (finite values; their outputs are not written).
constexpr int kQBlockHalves = kRowsPerBlock * kRep * kHeadDim;  // 32 KB
template <int RB, int NW>  // rows of the block: RB / (2 NW) instructions per wave
__device__ __forceinline__ void dma_q(u32x4v qr, int row0, int last_row, int ldq_bytes, const f16* qdst,
                                      int wave, int lane) {
    static_assert(RB % (2 * NW) == 0, "whole KBs per wave");
#pragma unroll
    for (int j = 0; j < RB / (2 * NW); ++j) {
        const int r = 2 * (NW * j + wave) + (lane >> 5);
        const int c = (lane & 31) ^ (r & 15);
        dma16(qr, min(row0 + r, last_row) * ldq_bytes + c * 16, lds_addr(qdst + (NW * j + wave) * 512));
    }
}

// 4 halves of V^T: ds_read_b64_tr_b16 transposes 16-bit elements within each
// 16-lane group (result lane 4m+e, element k <- source lane 4k+m, element e).
__device__ __forceinline__ half4v read_tr(const f16* p) {
    return __builtin_bit_cast(half4v, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)p));
}

// Per-wave state.
struct Wave {
    half8v qb[8];     // Q^T B operand, k-step ks: dims 16*ks + 8*g .. +8 of query n
    float16v o[4];    // O^T: o[db][i] = dim db*32 + 8*(i/4) + 4*g + i%4 of query n
    float m;          // running max the exponents are taken against
    float l;          // running row sum
    int kaddr[8];     // K operand of k-step ks, rows 0..31 of the half tile (halves)
    int vbase;        // V^T operand source address, slab 0, key 0 (halves)
    int g, qpos;
    float scale_log2;
};

// First half of a step over NB * 32 keys: S^T from K rows kt[0..32 NB - 1]
// (first key k0), row max, the running-max update, P^T (f16, B-operand
// layout) and its row sum.  MASK: some key is past some row's position.
template <bool MASK, int NB>
__device__ __forceinline__ void step_s(Wave& w, const f16* kt, int k0, half8v (&pb)[2 * NB]) {
    // S^T: keys kb*32 + (8*(i/4) + 4*g + i%4) x query n, accumulated over dims.
    float16v s[NB];
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) s[kb] = (float16v){};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int kb = 0; kb < NB; ++kb) {
            const half8v ka = *(const half8v*)&kt[kb * 32 * kHeadDim + w.kaddr[ks]];
            s[kb] = mfma32(ka, w.qb[ks], s[kb]);
        }
    // Operand reads run at most two k-steps ahead of the MFMAs (bounded
    // register lifetime; 8 NB reads + 8 NB MFMAs).
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * NB, 0);
#pragma unroll
    for (int i = 0; i < 6; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, NB, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, NB, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * NB, 0);
    float mx = kNegInf;
#pragma unroll
    for (int kb = 0; kb < NB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (MASK) {
                const int key = k0 + kb * 32 + 8 * (i >> 2) + 4 * w.g + (i & 3);
                s[kb][i] = key > w.qpos ? kNegInf : s[kb][i];
            }
            mx = fmaxf(mx, s[kb][i]);
        }
    mx = halves_max(mx) * w.scale_log2;
    // Move the running max when a row max passed it by more than the slack.
    {
        const bool up = mx > w.m + kRescaleSlack;
        if (__ballot(up)) {
            const float mn = up ? mx : w.m;
            const float alpha = w.m == kNegInf ? 0.0f : fast_exp2(w.m - mn);
#pragma unroll
            for (int db = 0; db < 4; ++db) w.o[db] *= alpha;
            w.l *= alpha;
            w.m = mn;
        }
    }
    const float mu = w.m == kNegInf ? 0.0f : w.m;
    // P^T = 2^(s*scale_log2 - m), k-step w4 covering keys 16*w4 + 4*g +
    // {0..3, 8..11}; the row sum from the same f16 values (v_dot2, f32 sum).
#pragma unroll
    for (int w4 = 0; w4 < 2 * NB; ++w4)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            pb[w4][j] = (f16)softmax_w_raw(s[w4 >> 1][8 * (w4 & 1) + j], w.scale_log2, mu);
    const half2v ones2 = {(f16)1.0f, (f16)1.0f};
    float ps = 0.0f;
#pragma unroll
    for (int w4 = 0; w4 < 2 * NB; ++w4)
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
            const half2v pr = {pb[w4][2 * q2], pb[w4][2 * q2 + 1]};
            ps = __builtin_amdgcn_fdot2(pr, ones2, ps, false);
        }
    w.l += halves_sum(ps);
}

// Second half: O^T += V^T P^T with V rows vt[0..32 NB - 1] (slab stride
// kTileKeys*32 halves).
template <int NB>
__device__ __forceinline__ void step_pv(Wave& w, const f16* vt, const half8v (&pb)[2 * NB]) {
#pragma unroll
    for (int w4 = 0; w4 < 2 * NB; ++w4)
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const f16* vp = vt + w.vbase + db * (kTileKeys * 32) + w4 * 16 * 32;
            const half4v lo = read_tr(vp);
            const half4v hi = read_tr(vp + 8 * 32);
            const half8v va = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            w.o[db] = mfma32(va, pb[w4], w.o[db]);
        }
    // Two transposing reads per MFMA, at most two MFMAs ahead.
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 8 * NB - 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
}

// Merge of the nsp split-K partials of one wave's 32 rows (lane = query row),
// for accumulator element chunks C0 .. C0+NC-1 (chunk k = elements 8k .. 8k+7
// = o[k / 2][8 (k % 2) .. +8]): returns the merged row sum and leaves the
// merged, unnormalised output in those chunks of o.  The partials are
// combined in split order whichever workgroup arrives last, so the result is
// bitwise reproducible.  Pass 1: the row max M (16 m values requested per
// memory round trip).  Pass 2: partials in groups of G, their (m, l) and, per
// 8-element chunk, the G x 8 accumulator values requested together.  Unused
// slots of a group read partial 0's record and drop it.
template <int G, int C0, int NC>
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
    float acc[NC][8];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[c][e] = 0.0f;
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
        for (int c = 0; c < NC; ++c) {
            float x[G][8];
#pragma unroll
            for (int u = 0; u < G; ++u) {
                const int i = i0 + u;
                const float* src =
                    ow + (int64_t)(i < nsp ? i : 0) * kPrefillItemFloats + (C0 + c) * 8 * 64;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float v = load_dev(src + e * 64);
                    x[u][e] = i < nsp ? v : 0.0f;
                }
            }
#pragma unroll
            for (int u = 0; u < G; ++u)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[c][e] = fmaf(x[u][e], w[u], acc[c][e]);
            __builtin_amdgcn_sched_barrier(0);  // keep the next chunk's loads after this one
        }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[(C0 + c) >> 1][8 * ((C0 + c) & 1) + e] = acc[c][e];
    return Ls;
}

// The same merge for nsp <= NP partials with every load -- (m, l) and the
// NC chunks of all NP records -- requested before the first use: one memory
// round trip instead of two plus one per chunk.  Unused slots read partial
// 0's record and weigh 0, and the sums run in the same order, so the result
// has the bits of merge_partials (whose unused slots add exact zeros).
template <int NP, int C0, int NC>
__device__ __forceinline__ float merge_partials_burst(const float* mlw, const float* ow, int nsp,
                                                      float16v (&o)[4]) {
    float mi[NP], li[NP], x[NC][NP][8];
#pragma unroll
    for (int u = 0; u < NP; ++u) {
        const float* rec = mlw + (int64_t)(u < nsp ? u : 0) * kPrefillItemMl;
        mi[u] = load_dev(rec);
        li[u] = load_dev(rec + 64);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int u = 0; u < NP; ++u) {
            const float* src = ow + (int64_t)(u < nsp ? u : 0) * kPrefillItemFloats + (C0 + c) * 8 * 64;
#pragma unroll
            for (int e = 0; e < 8; ++e) x[c][u][e] = load_dev(src + e * 64);
        }
    float M = kNegInf;
#pragma unroll
    for (int u = 0; u < NP; ++u) M = fmaxf(M, u < nsp ? mi[u] : kNegInf);
    float w[NP];
    float Ls = 0.0f;
#pragma unroll
    for (int u = 0; u < NP; ++u) {
        w[u] = (u >= nsp || mi[u] == kNegInf) ? 0.0f : fast_exp2(mi[u] - M);
        Ls = fmaf(u < nsp ? li[u] : 0.0f, w[u], Ls);
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll
        for (int u = 0; u < NP; ++u)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(u < nsp ? x[c][u][e] : 0.0f, w[u], acc[e]);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[(C0 + c) >> 1][8 * ((C0 + c) & 1) + e] = acc[e];
    }
    return Ls;
}

// Kernel state the epilogue needs.
// rec: this item's partial record; rec0: the record of split 0 of its (row
// block, kv head) (the splits' records follow it); ctr: their arrival counter.
struct EpiArgs {
    const PrefillArgs& a;
    float* ws_o;
    float* ws_ml;
    uint32_t* ctr;
    f16* K0;
    f16* K1;
    f16* V0;
    f16* V1;
    f16* Q;
    int64_t rec, rec0;
    int nsp, rw, r, head;
    bool row_ok;
    int g, lane, tid;
};

// Epilogue of a 32-row block (four key groups of 32 keys per row wave):
// wave (rw, KG) finishes dim block KG.  Each wave leaves its other three
// blocks (16 accumulator elements x 64 lanes, element-major) and its (m, l)
// in LDS -- the tile buffers and the free half of the Q block -- and
// combines the four partials of its block in key-group order.  A split key
// range then publishes the combined block (and KG 0 its (m, l)) and the last
// item to arrive merges the splits of its block.
template <int KG>
__device__ __forceinline__ void epilogue4(Wave& w, const EpiArgs& e) {
    const int lane = e.lane, rw = e.rw;
    // Partials of row wave rw, key group src: 16 KB at (rw ? V : K)(src >> 1)
    // + (src & 1) * 16 KB, dim block db at + db * 4 KB.
    auto blk = [&](int src, int db) {
        f16* b = rw ? (src < 2 ? e.V0 : e.V1) : (src < 2 ? e.K0 : e.K1);
        return reinterpret_cast<float*>(b) + (src & 1) * 4096 + db * 1024;
    };
    float* ml = reinterpret_cast<float*>(e.Q + kQBlockHalves / 2) + rw * 4 * 128;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
        if (db == KG) continue;
        float* dst = blk(KG, db);
#pragma unroll
        for (int i = 0; i < 16; ++i) dst[i * 64 + lane] = w.o[db][i];
    }
    ml[KG * 128 + lane] = w.m;
    ml[KG * 128 + 64 + lane] = w.l;
    __syncthreads();
    float mj[4], lj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mj[j] = j == KG ? w.m : ml[j * 128 + lane];
        lj[j] = j == KG ? w.l : ml[j * 128 + 64 + lane];
    }
    const float M = fmaxf(fmaxf(mj[0], mj[1]), fmaxf(mj[2], mj[3]));
    float L = 0.0f;
    float16v o = (float16v){};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float aj = mj[j] == kNegInf ? 0.0f : fast_exp2(mj[j] - M);
        L = fmaf(lj[j], aj, L);
        const float* src = blk(j, KG);
#pragma unroll
        for (int i = 0; i < 16; ++i) o[i] = fmaf(j == KG ? w.o[KG][i] : src[i * 64 + lane], aj, o[i]);
    }
    f16* orow = e.a.out + (int64_t)e.r * (e.a.nqh * kHeadDim) + e.head * kHeadDim;
    auto write_out = [&](const float16v& ob, float l) {
        if (!e.row_ok) return;
        const float inv = 1.0f / l;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            half4v h4;
#pragma unroll
            for (int x = 0; x < 4; ++x) h4[x] = (f16)(ob[q4 * 4 + x] * inv);
            *(half4v*)(orow + KG * 32 + 8 * q4 + 4 * e.g) = h4;
        }
    };
    if (e.nsp == 1) {
        write_out(o, L);
        return;
    }
    // Publish dim block KG of row wave rw (element-major, as the 64-row
    // epilogue's records), (m, l) from key group 0; then the ticket.
    {
        float* po = e.ws_o + e.rec * kPrefillItemFloats + rw * kPrefillWaveFloats;
#pragma unroll
        for (int i = 0; i < 16; ++i) store_dev(po + (KG * 16 + i) * 64 + lane, o[i]);
        if (KG == 0) {
            float* pml = e.ws_ml + e.rec * kPrefillItemMl + rw * kPrefillWaveMl;
            store_dev(pml + lane, M);
            store_dev(pml + 64 + lane, L);
        }
    }
    int& s_last = *reinterpret_cast<int*>(e.V0 + kTileHalves - 8);
    stores_done_barrier();
    if (e.tid == 0) s_last = (ticket_add(e.ctr) == (uint32_t)(e.nsp - 1));
    __syncthreads();
    if (!s_last) return;
    const float* mlw = e.ws_ml + e.rec0 * kPrefillItemMl + rw * kPrefillWaveMl + lane;
    const float* ow = e.ws_o + e.rec0 * kPrefillItemFloats + rw * kPrefillWaveFloats + lane;
    float16v om[4];
    const float Ls = e.nsp <= 2   ? merge_partials_burst<2, 2 * KG, 2>(mlw, ow, e.nsp, om)
                     : e.nsp <= 4 ? merge_partials_burst<4, 2 * KG, 2>(mlw, ow, e.nsp, om)
                                  : merge_partials<8, 2 * KG, 2>(mlw, ow, e.nsp, om);
    write_out(om[KG], Ls);
    if (e.tid == 0) ticket_reset(e.ctr);
}

// Epilogue of the wave of key group KG: wave (rw, KG) keeps dim blocks 2*KG
// and 2*KG+1 of the output and hands the other two blocks, with its (m, l),
// to its twin through LDS (element-major records: every access is 256
// contiguous bytes).  Then it writes, publishes and merges only its blocks.
template <int KG>
__device__ __forceinline__ void epilogue(Wave& w, const EpiArgs& e) {
    constexpr int kMine = 2 * KG, kTheirs = 2 * (KG ^ 1);
    const int lane = e.lane, rw = e.rw;
    float* xbase = reinterpret_cast<float*>(rw < 2 ? e.K0 : e.K1) + (rw & 1) * 2 * (32 * 64);
    float* xo_out = xbase + KG * (32 * 64);
    float* xo_in = xbase + (KG ^ 1) * (32 * 64);
    float* xml_out = reinterpret_cast<float*>(e.V1) + (rw * 2 + KG) * 128;
    float* xml_in = reinterpret_cast<float*>(e.V1) + (rw * 2 + (KG ^ 1)) * 128;
    int& s_last = *reinterpret_cast<int*>(e.V0);
    static_assert(2 * 2 * 32 * 64 * 4 <= kTileHalves * 2, "two row waves' halves per K buffer");
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int i = 0; i < 16; ++i) xo_out[(d * 16 + i) * 64 + lane] = w.o[kTheirs + d][i];
    xml_out[lane] = w.m;
    xml_out[64 + lane] = w.l;
    __syncthreads();
    {
        const float m1 = xml_in[lane], l1 = xml_in[64 + lane];
        const float M = fmaxf(w.m, m1);
        const float a0 = w.m == kNegInf ? 0.0f : fast_exp2(w.m - M);
        const float a1 = m1 == kNegInf ? 0.0f : fast_exp2(m1 - M);
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i)
                w.o[kMine + d][i] = w.o[kMine + d][i] * a0 + xo_in[(d * 16 + i) * 64 + lane] * a1;
        w.l = w.l * a0 + l1 * a1;
        w.m = M;
    }
    float16v (&o)[4] = w.o;

    // o[db][i] holds dim db*32 + 8*(i/4) + 4*g + i%4 of query row r.
    f16* orow = e.a.out + (int64_t)e.r * (e.a.nqh * kHeadDim) + e.head * kHeadDim;
    auto write_out = [&](float l) {
        if (!e.row_ok) return;
        const float inv = 1.0f / l;
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                half4v h4;
#pragma unroll
                for (int x = 0; x < 4; ++x) h4[x] = (f16)(o[kMine + d][q4 * 4 + x] * inv);
                *(half4v*)(orow + (kMine + d) * 32 + 8 * q4 + 4 * e.g) = h4;
            }
    };
    if (e.nsp == 1) {
        write_out(w.l);
        return;
    }

    // Partial of this row wave: 64 accumulator elements x 64 lanes,
    // element-major (element x of lane l at [x][l]), each wave of the pair
    // storing its 32; then (m, l) per lane.  Published with device-scope
    // stores (see stores_done_barrier).
    {
        float* po = e.ws_o + e.rec * kPrefillItemFloats + rw * kPrefillWaveFloats;
#pragma unroll
        for (int d = 0; d < 2; ++d)
#pragma unroll
            for (int i = 0; i < 16; ++i) store_dev(po + ((kMine + d) * 16 + i) * 64 + lane, o[kMine + d][i]);
        if (KG == 0) {
            float* pml = e.ws_ml + e.rec * kPrefillItemMl + rw * kPrefillWaveMl;
            store_dev(pml + lane, w.m);
            store_dev(pml + 64 + lane, w.l);
        }
    }
    stores_done_barrier();
    if (e.tid == 0) s_last = (ticket_add(e.ctr) == (uint32_t)(e.nsp - 1));
    __syncthreads();
    if (!s_last) return;

    // Last arrival: merge the nsp partials of this (kv head, row block); each
    // wave merges its half of its row wave's 32 rows.
    const float* mlw = e.ws_ml + e.rec0 * kPrefillItemMl + rw * kPrefillWaveMl + lane;
    const float* ow = e.ws_o + e.rec0 * kPrefillItemFloats + rw * kPrefillWaveFloats + lane;
    const float Ls = e.nsp <= 2   ? merge_partials_burst<2, 4 * KG, 4>(mlw, ow, e.nsp, o)
                     : e.nsp <= 4 ? merge_partials_burst<4, 4 * KG, 4>(mlw, ow, e.nsp, o)
                                  : merge_partials<8, 4 * KG, 4>(mlw, ow, e.nsp, o);
    write_out(Ls);
    if (e.tid == 0) ticket_reset(e.ctr);
}

// NKG = 2: 64-row blocks, row wave rw = wave & 3 (2 q heads x 2 x 32 rows),
// key group kg = wave >> 2 taking keys 64 kg .. +64 of every tile.  NKG = 4
// (short key ranges): 32-row blocks, rw = wave & 1 (the 2 q heads), kg =
// wave >> 1 taking keys 32 kg .. +32 -- half the work per workgroup and
// twice the workgroups.  NKG = 4 on NW = 4 waves: 16-row blocks, one row
// wave whose 32 MFMA columns hold both q heads (column n: head n / 16, row
// n % 16) and kg = wave -- one wave per SIMD, a quarter of the 64-row
// block's work per workgroup.  SLICE (16-row blocks only): each wave copies
// the keys it reads and the loop has no barrier (dma_slice).
template <int NKG, int NW = kAllWaves, bool SLICE = false>
__global__ __launch_bounds__(NW * 64, 1) void prefill_attn_kernel(
    PrefillArgs a, PrefillSegs S, float* __restrict__ ws_o, float* __restrict__ ws_ml,
    uint32_t* __restrict__ counters) {
    // 160 KB: K and V tiles, double buffered, and the Q block.
    __shared__ __attribute__((aligned(16))) f16 K0[kTileHalves];
    __shared__ __attribute__((aligned(16))) f16 K1[kTileHalves];
    __shared__ __attribute__((aligned(16))) f16 V0[kTileHalves];
    __shared__ __attribute__((aligned(16))) f16 V1[kTileHalves];
    __shared__ __attribute__((aligned(16))) f16 Qs[kQBlockHalves];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    static_assert(NW == kAllWaves || (NW == 4 && NKG == 4), "wave counts");
    static_assert(!SLICE || NW == 4, "per-wave copies: 16-row blocks");
    constexpr int kRowWaves = NW / NKG;
    constexpr int RB = 16 * kRowWaves;        // rows per block: 64, 32 or 16
    constexpr bool PACK = kRowWaves == 1;     // both q heads in one wave's columns
    static_assert(!PACK || kRep == 2, "two q heads x 16 rows fill a wave's 32 MFMA columns");
    constexpr int GK = kTileKeys / NKG;       // keys per key group and tile: 64 or 32
    constexpr int NB = GK / 32;               // 32-key MFMA blocks per step
    const int wave = tid >> 6;       // 0..7: copy slot
    // The same index in a scalar register, for the copies' LDS addresses
    // (M0 then comes from scalar arithmetic instead of a readfirstlane of a
    // vector address per copy).
    const int cwave = __builtin_amdgcn_readfirstlane(wave);
    const int rw = wave % kRowWaves; // row wave
    const int kg = wave / kRowWaves; // key group
    const int n = lane & 31;  // query column within the wave's 32 rows
    const int g = lane >> 5;  // k-slot group of the MFMA operands

    // Piece = number of later piece starts at or before this workgroup (one
    // lane per piece, a ballot); then kv head minor, and the row block from
    // the piece's item table (one lane per row block, a ballot).  Each lookup
    // is one round trip: lane i reads piece i's fields (the argument arrays
    // hold 64 pieces) and then row block i's table entries (indices clamped
    // to the piece's nrb, inside its table), and the chosen piece's and row
    // block's fields are lane reads, not further dependent loads.
    static_assert(kMaxPrefillPieces == 64 && kMaxRowBlocks <= 64, "one lane per piece / row block");
    const int p_ib0 = S.item_base[lane], p_ib1 = S.item_base[lane + 1], p_part = S.part_base[lane];
    const int p_rbb = S.rb_base[lane], p_nrb = S.nrb[lane], p_tps = S.tps[lane];
    const int p_ks = S.kv_start[lane], p_rows = S.rows[lane], p_rowb = S.row_base[lane];
    const int64_t p_kvo = S.kv_off[lane];
    // Loaded with the others (not under the lane + 1 < S.n test), and the
    // argument pointers with them (not after the second lookup).
    asm volatile("" ::"v"(p_ib1), "s"(a.q), "s"(a.out), "s"(a.k), "s"(a.v));
    const int pc = __popcll(__ballot(lane + 1 < S.n && p_ib1 <= (int)blockIdx.x));
    const int local = blockIdx.x - __builtin_amdgcn_readlane(p_ib0, pc);
    const int kvh = local % a.nkvh;
    const int rem = local / a.nkvh;
    const int rb_base = __builtin_amdgcn_readlane(p_rbb, pc);
    const int nrb = __builtin_amdgcn_readlane(p_nrb, pc);
    // A piece with one item per row block (no split) needs no item table:
    // its row block is the item.  Otherwise a second round trip reads it.
    const int pitems = __builtin_amdgcn_readlane(p_ib1, pc) - __builtin_amdgcn_readlane(p_ib0, pc);
    int rb = rem, sp_rb = rem, nsp = 1, sp_nrb = nrb;
    if (pitems != a.nkvh * nrb) {
        const int* sp = S.sp + rb_base + pc;
        const int sp0 = sp[min(lane, nrb)], sp1 = sp[min(lane + 1, nrb)];
        rb = __popcll(__ballot(lane + 1 < nrb && sp1 <= rem));
        sp_rb = __builtin_amdgcn_readlane(sp0, rb);
        nsp = __builtin_amdgcn_readlane(sp1, rb) - sp_rb;
        sp_nrb = __builtin_amdgcn_readlane(sp1, nrb - 1);
    }
    const int split = rem - sp_rb;
    const int tps = __builtin_amdgcn_readlane(p_tps, pc);
    const int64_t rec0 = (int64_t)__builtin_amdgcn_readlane(p_part, pc) + (int64_t)kvh * sp_nrb + sp_rb;
    uint32_t* ctr = counters + (int64_t)(rb_base + rb) * a.nkvh + kvh;
    a.s = __builtin_amdgcn_readlane(p_rows, pc);
    a.kv_start = __builtin_amdgcn_readlane(p_ks, pc);
    const int row_base = __builtin_amdgcn_readlane(p_rowb, pc);
    const int64_t kv_off = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(p_kvo >> 32), pc) << 32) |
                                     (uint32_t)__builtin_amdgcn_readlane((int)p_kvo, pc));
    a.q += (int64_t)row_base * a.nqh * kHeadDim;
    a.out += (int64_t)row_base * a.nqh * kHeadDim;
    a.k += kv_off;
    a.v += kv_off;
    const int row0 = rb * RB;
    const int kend = a.kv_start + min(row0 + RB, a.s);  // keys < kend
    const int ntiles = (kend + kTileKeys - 1) / kTileKeys;
    const int t_begin = split * tps;
    const int t_end = min(t_begin + tps, ntiles);

    // This lane's q head (of the kv head's kRep) and row within the block.
    const int hsel = PACK ? (n >> 4) : (rw & 1);
    const int rin = PACK ? (n & 15) : (rw >> 1) * 32 + n;
    const int head = kvh * kRep + hsel;
    const int wrow0 = row0 + (PACK ? 0 : (rw >> 1) * 32);  // first row of this wave
    const int r = row0 + rin;                   // this lane's query row
    const bool row_ok = r < a.s;
    const int ldq = a.nqh * kHeadDim;
    // Key range of the wave's rows: a half tile from key k0 on is masked when
    // k0 + 63 > first_pos and skipped when k0 > last_pos.
    const int first_pos = a.kv_start + wrow0;
    const int last_pos = first_pos + (PACK ? 15 : 31);

    const u32x4v kres = make_rsrc_words(a.k + kvh * a.head_stride, kend * kHeadDim * 2);
    const u32x4v vres = make_rsrc_words(a.v + kvh * a.head_stride, kend * kHeadDim * 2);
    // This thread's copy slots (see the layout notes above dma16).
    const int krow = 4 * wave + (lane >> 4);
    const int kchunk = ((lane & 15) ^ swz16(krow)) * 16;
    const int vrow = 16 * wave + (lane >> 2);
    const int vchunk = (lane & 3) * 16;

    // Every copy is issued here in this order and waited for by count:
    // tile t_begin (kTileCopies<NW> per thread), the Q block, tile t_begin + 1.
    const u32x4v qres = make_rsrc_words(a.q + kvh * kRep * kHeadDim,
                                        (a.s - 1) * ldq * 2 + kRep * kHeadDim * 2);
    auto copy_tile = [&](int t, const f16* kt, const f16* vt) {
        if constexpr (SLICE)
            dma_slice(kres, vres, t * kTileKeys, kend, kt, vt, cwave, lane);
        else
            dma_tile<NW>(kres, vres, t * kTileKeys, kend, krow, kchunk, vrow, vchunk, kt, vt, cwave);
    };
    copy_tile(t_begin, K0, V0);
    dma_q<RB, NW>(qres, row0, a.s - 1, ldq * 2, Qs, cwave, lane);
    const bool two = t_begin + 1 < t_end;
    if (two) copy_tile(t_begin + 1, K1, V1);

    Wave w;
    w.g = g;
    w.qpos = a.kv_start + r;
    w.scale_log2 = a.scale_log2;
#pragma unroll
    for (int db = 0; db < 4; ++db) w.o[db] = (float16v){};
    w.m = kNegInf;
    w.l = 0.0f;
    // K operand of k-step ks: row n, chunk 2*ks + g; V^T operand: source lane
    // 16*q4 + 4*k + m reads row 4*(q4>>1) + k, dims 16*(q4&1) + 4*m .. +3.
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) w.kaddr[ks] = n * kHeadDim + (((2 * ks + g) ^ swz16(n)) * 8);
    {
        const int q4 = lane >> 4;
        w.vbase = (4 * (q4 >> 1) + ((lane >> 2) & 3)) * 32 + 16 * (q4 & 1) + 4 * (lane & 3);
    }

    // This thread's copies of the next tile have landed (the only ones
    // outstanding), then every wave's have.
    auto tile_sync = [&]() {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __syncthreads();
    };
    // Tile t: this wave's half of it (tile t+1 is in flight meanwhile), then
    // once every wave is done with its buffers and tile t+1 has landed, the
    // copy of tile t+2 into them.  Two tiles per iteration, so every LDS
    // address is a per-lane base plus a constant.
    // SLICE: each wave reads and copies only its own key group's rows
    // (dma_slice), so it waits for its own copies of tile t (those of tile
    // t + 1 may stay in flight) and, once its own reads of the buffers have
    // returned, copies tile t + 2 into them, with no barrier.
    auto run = [&](const f16* kt, const f16* vt, int t) {
        if constexpr (SLICE) {
            static_assert(kTileCopies<NW> == 16, "vmcnt(16) below");
            if (t + 1 < t_end)
                asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        const int k0 = t * kTileKeys + kg * GK;
        if (k0 <= last_pos) {  // some key visible to some row
            const f16* kh = kt + kg * GK * kHeadDim;
            const f16* vh = vt + kg * GK * 32;
            half8v pb[2 * NB];
            if (k0 + GK - 1 <= first_pos)  // no key masked
                step_s<false, NB>(w, kh, k0, pb);
            else
                step_s<true, NB>(w, kh, k0, pb);
            step_pv<NB>(w, vh, pb);
        }
        if constexpr (SLICE) {
            if (t + 2 < t_end) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                copy_tile(t + 2, kt, vt);
            }
        } else {
            tile_sync();
            if (t + 2 < t_end) copy_tile(t + 2, kt, vt);
        }
    };
    // Tile t_begin and Q have landed (tile t_begin + 1 may be in flight).
    static_assert(kTileCopies<NW> == 8 || kTileCopies<NW> == 16, "vmcnt encodings below");
    if (two) {
        if constexpr (kTileCopies<NW> == 8)
            __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
        else
            __builtin_amdgcn_s_waitcnt(0x4F70);  // vmcnt(16)
    } else {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    __syncthreads();
    {
        // Q^T operand, k-step ks: chunk 16*hsel + 2*ks + g of the lane's row.
        const int qr = rin;
        const f16* qrow = Qs + qr * (kRep * kHeadDim);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
            const int c = ((hsel * 16 + 2 * ks + g) ^ (qr & 15));
            w.qb[ks] = *(const half8v*)(qrow + c * 8);
        }
    }
    for (int t = t_begin;;) {
        run(K0, V0, t);
        if (++t >= t_end) break;
        run(K1, V1, t);
        if (++t >= t_end) break;
    }

    // The two key groups of a row wave combine through LDS (the tile buffers
    // are free now); from here on both waves of a pair share the epilogue
    // work half and half.
    EpiArgs e{a, ws_o, ws_ml, ctr, K0, K1, V0, V1, Qs, rec0 + split, rec0, nsp, rw, r, head, row_ok, g, lane, tid};
    // Every wave is done with the tile buffers (the SLICE loop has no
    // barrier) and has no copy in flight (its last tile waited for vmcnt(0)).
    if constexpr (SLICE) __syncthreads();
    if constexpr (NKG == 2) {
        if (kg == 0)
            epilogue<0>(w, e);
        else
            epilogue<1>(w, e);
    } else {
        switch (kg) {
            case 0: epilogue4<0>(w, e); break;
            case 1: epilogue4<1>(w, e); break;
            case 2: epilogue4<2>(w, e); break;
            default: epilogue4<3>(w, e); break;
        }
    }
}

}  // namespace

PrefillPlan plan_prefill(int s, int kv_start, int nkvh, int tiles_per_split, int rows_per_block) {
    PrefillPlan P{};
    P.rows_per_block = rows_per_block;
    P.nrb = (s + rows_per_block - 1) / rows_per_block;
    P.tps = tiles_per_split;
    P.sp_base[0] = 0;
    for (int rb = 0; rb < P.nrb; ++rb) {
        const int kend = kv_start + std::min((rb + 1) * rows_per_block, s);
        const int ntiles = (kend + kTileKeys - 1) / kTileKeys;
        P.sp_base[rb + 1] = P.sp_base[rb] + (ntiles + P.tps - 1) / P.tps;
    }
    P.items_per_kvh = P.sp_base[P.nrb];
    (void)nkvh;
    return P;
}

hipError_t launch_prefill_attn(const PrefillArgs& a, int rows_per_block, const PrefillSegs& S,
                               const PrefillWs& ws, hipStream_t stream) {
    if (S.n <= 0 || S.n > kMaxPrefillPieces) return hipErrorInvalidValue;
    const int items = S.item_base[S.n];
    if (items <= 0) return hipSuccess;
    const int last = S.n - 1;
    const int rbs = S.rb_base[last] + S.nrb[last];
    const int64_t recs = (int64_t)S.part_base[last] + (int64_t)a.nkvh * S.sp[S.rb_base[last] + last + S.nrb[last]];
    if (rbs > kMaxLaunchRowBlocks || recs > ws.items) return hipErrorInvalidValue;
    // 16-row blocks (never split): the per-wave copy loop once some item has
    // more than 4 tiles (at 8 tiles 11.2 against 11.9 us; up to 4 tiles
    // about 0.05 us slower than the barrier loop, whose copies keep up).
    int max_tiles = 0;
    for (int p = 0; p < S.n; ++p)
        max_tiles = std::max(max_tiles, (S.kv_start[p] + S.rows[p] + kTileKeys - 1) / kTileKeys);
    if (rows_per_block == kRowsPerBlock / 4 && max_tiles > 4)
        hipLaunchKernelGGL((prefill_attn_kernel<4, 4, true>), dim3(items), dim3(4 * 64), 0, stream, a, S,
                           ws.o, ws.ml, ws.counters);
    else if (rows_per_block == kRowsPerBlock / 4)
        hipLaunchKernelGGL((prefill_attn_kernel<4, 4>), dim3(items), dim3(4 * 64), 0, stream, a, S,
                           ws.o, ws.ml, ws.counters);
    else if (rows_per_block == kRowsPerBlock / 2)
        hipLaunchKernelGGL((prefill_attn_kernel<4>), dim3(items), dim3(kThreads), 0, stream, a, S,
                           ws.o, ws.ml, ws.counters);
    else if (rows_per_block == kRowsPerBlock)
        hipLaunchKernelGGL((prefill_attn_kernel<2>), dim3(items), dim3(kThreads), 0, stream, a, S,
                           ws.o, ws.ml, ws.counters);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace qasr
