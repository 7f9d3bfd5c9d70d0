// kernels.hpp -- launch-plan structs and launchers shared by the C ABI
// (qasr_attn.hip) and the kernel translation units.
#pragma once

#include "common.hpp"

namespace qasr {

// Where one KV pool lives: element (slot, layer, kv, head, pos, d) is at
// base + slot*slot_stride + layer*layer_stride + kv*kv_stride + head*head_stride
//      + pos*kHeadDim + d.
struct CacheGeom {
    f16* base;
    int64_t slot_stride;
    int64_t layer_stride;
    int64_t kv_stride;
    int64_t head_stride;
    int32_t nkvh;
    int32_t cap;
};

// Stage (a) plan: up to kMaxBatch segments of consecutive rows.
struct SegPlan {
    int32_t nseg;
    int32_t nqh;
    float eps;
    int32_t slot[kMaxBatch];
    int32_t pos0[kMaxBatch];
    int32_t row_base[kMaxBatch + 1];  // prefix sum of rows; row_base[nseg] = total
};

// Stage (b) plan.  Entry b's keys are cut into granules of gran[b] keys (a
// multiple of kDecodeGranuleQuantum, a function of len[b] only, at most
// kDecodeMaxGranules of them); a workgroup runs `run[b]` consecutive granules
// of one kv head, runs aligned to the entry's end (the first takes any
// remainder).  Workgroups of entry b are wg_base[b] .. wg_base[b+1]-1, kv
// head minor; the partial record of (entry b, kv head h, granule i) is
// part_base[b] + h * ceil(len[b] / gran[b]) + i.
struct DecodePlan {
    int32_t batch;
    int32_t nqh;
    float scale_log2;  // softmax scale * log2(e): scores live in the exp2 domain
    float eps;
    int32_t slot[kMaxBatch];
    int32_t len[kMaxBatch];    // keys attended; the fused step appends key len-1
    int32_t gran[kMaxBatch];   // keys per granule
    int32_t run[kMaxBatch];    // granules per workgroup
    int32_t wg_base[kMaxBatch + 1];
    int32_t part_base[kMaxBatch + 1];
};

constexpr int kDecodeWaves = 4;       // workgroup size (waves)
constexpr int kDecodeWavesPerEU = 2;  // occupancy target: <= 256 VGPRs (two pass buffers)
constexpr int kDecodeTileKeys = 32;   // keys per wave pass
constexpr int kDecodeWgKeys = kDecodeWaves * kDecodeTileKeys;  // keys per workgroup pass
constexpr int kDecodeGranuleQuantum = 2 * kDecodeWgKeys;        // granules are multiples of this
constexpr int kDecodeMaxGranules = 32;  // granules per entry: the merge reads them in one round trip
constexpr int kDecodeMaxRunGranules = 8;  // granules of one workgroup's run (wave partials in LDS)

// Split-K workspace of one launch: per granule partial the unnormalised
// output of both q heads (2 x 128 f32) and (max, sum) per head, plus one
// arrival counter per (batch entry, kv head).  Counters start at zero and the
// merging workgroup puts them back to zero.
struct DecodeWs {
    float* acc;         // [items][2][128]
    float* ml;          // [items][4]: m0, m1, l0, l1
    uint32_t* counters; // [kMaxBatch * nkvh]
    int64_t items;
};

hipError_t launch_norm_rope_append(const CacheGeom& g, int layer, const SegPlan& P,
                                   const f16* qkv, const f16* q_gain, const f16* k_gain,
                                   const f16* cos_tab, const f16* sin_tab, f16* q_out,
                                   hipStream_t stream);

hipError_t launch_decode_attn(bool fused, const CacheGeom& g, int layer, const DecodePlan& P,
                              int total_wgs, const f16* q_or_qkv, const f16* q_gain,
                              const f16* k_gain, const f16* cos_tab, const f16* sin_tab, f16* out,
                              const DecodeWs& ws, hipStream_t stream);

struct PrefillArgs {
    const f16* q;   // [s][nqh*128], roped
    f16* out;       // [s][nqh*128]
    const f16* k;   // K block of (slot, layer): [nkvh][cap][128]
    const f16* v;   // V block
    int64_t head_stride;
    int32_t nqh;
    int32_t nkvh;
    int32_t s;
    int32_t kv_start;
    float scale_log2;
};

// Stage (c).  A prefill is cut into pieces of at most kMaxRowBlocks * 64
// consecutive rows of one segment.  A piece's plan is a function of its rows
// and first position only (choose_prefill_plan on the host): row blocks of 64
// rows (32 for unsplit short key ranges), and each row block's 128-key tiles
// split into pieces of `tps` tiles.  So a prompt's bits do not depend on what
// else the launch carries: the one-segment entry point and the batched one
// run the same items.
constexpr int kMaxRowBlocks = 64;  // row blocks of one piece (4096 rows)
constexpr int kPrefillRows = 64;
struct PrefillPlan {
    int32_t rows_per_block;  // kPrefillRows, or kPrefillRows / 2 or / 4 for unsplit short key ranges
    int32_t nrb;
    int32_t tps;
    int32_t items_per_kvh;
    int32_t sp_base[kMaxRowBlocks + 1];  // row block rb's items of a kv head: sp_base[rb] ..
};

// Split workspace: per item 4 waves x (64 accumulator elements x 64 lanes of
// unnormalised O, element-major; then m and l per lane) -- a 32-row item uses
// half of it; one arrival counter per (row block of the launch, kv head),
// zero at rest.
struct PrefillWs {
    float* o;
    float* ml;
    uint32_t* counters;  // [kMaxLaunchRowBlocks * nkvh]
    int64_t items;
};
constexpr int kPrefillWaves = 4;      // waves that own rows (2 q heads x 2 x 32 rows)
constexpr int kPrefillKeyGroups = 2;  // each row wave has a twin taking the other half of every tile
constexpr int kPrefillTileKeys = 128;
constexpr int64_t kPrefillWaveFloats = 64 * 64;  // 64 accumulator elements x 64 lanes
constexpr int64_t kPrefillWaveMl = 2 * 64;       // m and l of each lane
constexpr int64_t kPrefillItemFloats = kPrefillWaves * kPrefillWaveFloats;
constexpr int64_t kPrefillItemMl = kPrefillWaves * kPrefillWaveMl;

// One launch: up to kMaxPrefillPieces pieces of one row block size.  Piece
// i: rows[i] q/out rows from row_base[i] at positions kv_start[i] ..; its K/V
// blocks start kv_off[i] elements past PrefillArgs::k / ::v; nrb[i] row
// blocks and tps[i] tiles per split; sp[sp_off(i) + rb] (sp_off(i) =
// rb_base[i] + i) is row block rb's first item within a kv head and
// sp[sp_off(i) + nrb[i]] the items per kv head.  Its workgroups are
// item_base[i] .. item_base[i+1]-1 (kv head minor, then row block, then
// split); its partial records part_base[i] + kvh * items_per_kvh + item; the
// arrival counter of (row block rb, kv head h) is (rb_base[i] + rb) * nkvh + h.
constexpr int kMaxPrefillPieces = 64;
constexpr int kMaxLaunchRowBlocks = 192;
struct PrefillSegs {
    int32_t n;
    int32_t item_base[kMaxPrefillPieces + 1];
    int32_t part_base[kMaxPrefillPieces];
    int32_t rb_base[kMaxPrefillPieces];
    int32_t nrb[kMaxPrefillPieces];
    int32_t tps[kMaxPrefillPieces];
    int32_t kv_start[kMaxPrefillPieces];
    int32_t rows[kMaxPrefillPieces];
    int32_t row_base[kMaxPrefillPieces];
    int64_t kv_off[kMaxPrefillPieces];
    int32_t sp[kMaxLaunchRowBlocks + kMaxPrefillPieces];
};

PrefillPlan plan_prefill(int s, int kv_start, int nkvh, int tiles_per_split,
                         int rows_per_block = kPrefillRows);
// rows_per_block: 64, 32 or 16, the block size every piece of S was planned with.
hipError_t launch_prefill_attn(const PrefillArgs& a, int rows_per_block, const PrefillSegs& S,
                               const PrefillWs& ws, hipStream_t stream);

// Prefill projections (gemm.hip): C[M][N] = f16(A[M][K] . B[N][K]^T (+ C)),
// f32 accumulation, row-major, leading dimensions K, K and N, 16-byte
// aligned.  gemm_f16_fits: K % 64 == 0, N % 256 == 0, both operands < 2 GB.
bool gemm_f16_fits(int M, int N, int K);
hipError_t launch_gemm_f16(const f16* A, const f16* B, f16* C, int M, int N, int K, bool accumulate,
                           int cus, hipStream_t stream);

}  // namespace qasr
