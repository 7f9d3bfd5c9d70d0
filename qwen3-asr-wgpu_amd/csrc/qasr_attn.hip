// qasr_attn.hip -- the C ABI (include/qasr_attn.h): contexts, KV pools, RoPE
// tables, argument checking, launch planning and dispatch of the stage (a),
// (b) and (c) kernels.
//
// Host-side mirror of the reference's attention plumbing inside
// WgpuTextDecoder (src/decoder.rs): load-time buffers (977-1246),
// ensure_capacity (1604-1661), set_rope_tables (1664-1667), per-step planning
// (1674-1714, 1932-2025, 3348-3451) and the prefill attention block
// (4856-5098).  Errors follow the reference's bounds checks
// (src/cpu_decoder.rs:489-495, 520; src/decoder.rs:4500-4530) but come back as
// status codes.

#include "qasr_attn.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <mutex>
#include <string>
#include <vector>

#include "abi_internal.hpp"
#include "kernels.hpp"

using qasr::f16;
using qasr_abi::DeviceScope;
using qasr_abi::fail;
using qasr_abi::g_err;
using qasr_abi::hip_fail;

namespace {

// f32 -> IEEE binary16 bits, round to nearest even, subnormals kept: the
// conversion of half::f16::from_f32 (inference.rs:1046-1047).  Written out on
// the bit level because the host pass's _Float16 cast is not RNE-exact.
uint16_t f16_bits(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);
    const int e = (int)(ax >> 23) - 127;
    uint32_t m = ax & 0x7fffffu;
    if (e >= -14) {
        uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
        const uint32_t rem = m & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
        return (uint16_t)(sign | h);
    }
    if (e < -25) return sign;
    m |= 0x800000u;
    const int shift = -e - 1;
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

// Positions a context may address (max_seq) and the planners accept: far
// past any KV pool that fits a GPU, small enough that no position, key or
// tile count of a plan overflows 32 bits.
constexpr int kMaxPositions = 1 << 24;

int env_int(const char* name, int dflt) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    return std::atoi(v);
}

}  // namespace

namespace {

qasr::CacheGeom geom(const qasr_kv* kv) {
    const qasr_attn_cfg& c = kv->ctx->cfg;
    qasr::CacheGeom g;
    g.base = kv->base;
    g.head_stride = (int64_t)kv->cap * qasr::kHeadDim;
    g.kv_stride = g.head_stride * c.num_key_value_heads;
    g.layer_stride = 2 * g.kv_stride;
    g.slot_stride = g.layer_stride * c.num_hidden_layers;
    g.nkvh = c.num_key_value_heads;
    g.cap = kv->cap;
    return g;
}

int target_cap(int need, int cap, int max_seq) {
    int64_t t = ((int64_t)need + QASR_KV_STEP - 1) / QASR_KV_STEP * QASR_KV_STEP;
    t = std::min<int64_t>(t, max_seq);
    t = std::max<int64_t>(t, cap);
    return (int)t;
}

void free_decode_ws(qasr_kv* kv) {
    if (kv->dws_acc) (void)hipFree(kv->dws_acc);
    if (kv->dws_ml) (void)hipFree(kv->dws_ml);
    if (kv->dws_ctr) (void)hipFree(kv->dws_ctr);
    kv->dws_acc = kv->dws_ml = nullptr;
    kv->dws_ctr = nullptr;
    kv->dws_items = 0;
}

void free_prefill_ws(qasr_kv* kv) {
    if (kv->pws_o) (void)hipFree(kv->pws_o);
    if (kv->pws_ml) (void)hipFree(kv->pws_ml);
    if (kv->pws_ctr) (void)hipFree(kv->pws_ctr);
    kv->pws_o = kv->pws_ml = nullptr;
    kv->pws_ctr = nullptr;
    kv->pws_items = 0;
}

// Decode workspace: one partial per granule of a launch (at most kMaxBatch
// entries x nkvh x kDecodeMaxGranules) and one ticket per (entry, kv head).
int alloc_decode_ws(qasr_kv* kv) {
    const int nkvh = kv->ctx->cfg.num_key_value_heads;
    const int64_t items = (int64_t)qasr::kMaxBatch * nkvh * qasr::kDecodeMaxGranules;
    HIP_TRY(hipMalloc(&kv->dws_acc, items * 2 * qasr::kHeadDim * sizeof(float)), "decode workspace");
    HIP_TRY(hipMalloc(&kv->dws_ml, items * 4 * sizeof(float)), "decode workspace");
    const size_t cbytes = (size_t)qasr::kMaxBatch * nkvh * sizeof(uint32_t);
    HIP_TRY(hipMalloc(&kv->dws_ctr, cbytes), "decode counters");
    HIP_TRY(hipMemset(kv->dws_ctr, 0, cbytes), "decode counters");
    kv->dws_items = items;
    return QASR_OK;
}

int ensure_prefill_ws(qasr_kv* kv, int64_t items) {
    if (items <= kv->pws_items) return QASR_OK;
    HIP_TRY(hipDeviceSynchronize(), "prefill workspace sync");
    free_prefill_ws(kv);
    const int nkvh = kv->ctx->cfg.num_key_value_heads;
    HIP_TRY(hipMalloc(&kv->pws_o, items * qasr::kPrefillItemFloats * sizeof(float)),
            "prefill workspace");
    HIP_TRY(hipMalloc(&kv->pws_ml, items * qasr::kPrefillItemMl * sizeof(float)),
            "prefill workspace");
    const size_t cbytes = (size_t)nkvh * qasr::kMaxLaunchRowBlocks * sizeof(uint32_t);
    HIP_TRY(hipMalloc(&kv->pws_ctr, cbytes), "prefill counters");
    HIP_TRY(hipMemset(kv->pws_ctr, 0, cbytes), "prefill counters");
    kv->pws_items = items;
    return QASR_OK;
}

// Decode launch plan, in two parts.
//
// 1. Granules: entry b's keys are cut into granules of G(len[b]) keys, a
//    multiple of 256 (two workgroup passes) leaving at most
//    QASR_DECODE_MAX_GRANULES (default and limit 32) granules: by default
//    256 keys up to 1024 keys, 1024 up to 8192, then len / 32 (granule_keys);
//    with QASR_DECODE_GRANULE = g, at least g keys.  Every granule
//    yields one partial and the partials merge in granule order, so an
//    entry's output bits are a function of its own length and keys: batch
//    composition, slot order and the device's CU count never change them
//    (the reference's --batch N == --batch 1, decoder.rs:1930-1931).
// 2. Runs: which workgroup runs which granules.  A workgroup takes `run`
//    consecutive granules (at most kDecodeMaxRunGranules) of one (entry, kv
//    head).  One CU streams at most
//    ~50-75 GB/s, so a launch runs at HBM rate only while most CUs stream:
//    the plan aims at QASR_DECODE_WGS workgroups (default one per CU) that
//    carry about the same number of keys.  When the batch leaves room
//    (entries x kv heads below the budget), the smallest per-workgroup key
//    budget C (a multiple of 256) is found for which runs of floor(C / G)
//    granules (at least one) fit the budget.  Batches at or past the budget
//    start from one workgroup per (entry, kv head) and split the run with
//    the most keys while it exceeds 1.5x the average keys per workgroup; the
//    extra workgroups run as the first ones finish.
int granule_keys(int L, int gmin, int gmax) {
    const int64_t q = qasr::kDecodeGranuleQuantum;
    int64_t want;
    if (gmin > 0) {
        want = std::max<int64_t>(gmin, ((int64_t)L + gmax - 1) / gmax);
    } else {
        // Default rule.  A granule costs a per-wave merge inside the stream
        // and a partial in the final merge, so entries of a batch want few,
        // large granules (config 3, 16 slots of 400-2400 keys: 21.0 us per
        // layer at 1024 keys, 22.4 at 512, 23.4 at 256); a lone entry wants
        // enough granules to spread over the GPU (one slot at 512 keys: 9.4 us
        // at 256, 10.6 at 1024; at 8193 keys: 13.6 us at 512, 17.8 at 1024).
        // So: 256 keys up to 1024 keys, 1024 up to 8192, and beyond that as
        // many granules as the merge takes (512 keys up to 16384).
        want = L <= 1024 ? 256 : L <= 8192 ? 1024 : ((int64_t)L + gmax - 1) / gmax;
    }
    return (int)((want + q - 1) / q * q);
}

int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Keys of one workgroup's run at most: its K/V buffer ranges stay below 1 GB.
constexpr int kMaxRunKeys = 1 << 22;

void plan_decode_granules(qasr::DecodePlan& P, int nkvh, int cus) {
    const int target = std::max(1, std::min(env_int("QASR_DECODE_WGS", cus), 8192));
    const int genv = env_int("QASR_DECODE_GRANULE", 0);  // > 0: max(this, len / max granules)
    const int gmin = genv > 0 ? std::max(qasr::kDecodeGranuleQuantum, genv) : 0;
    const int gmax = std::max(1, std::min(env_int("QASR_DECODE_MAX_GRANULES", qasr::kDecodeMaxGranules),
                                          qasr::kDecodeMaxGranules));
    int ngr[qasr::kMaxBatch], run[qasr::kMaxBatch];
    int64_t keys = 0;
    int pairs = 0;
    for (int i = 0; i < P.batch; ++i) {
        P.gran[i] = granule_keys(P.len[i], gmin, gmax);
        ngr[i] = ceil_div(P.len[i], P.gran[i]);
        run[i] = std::max(1, std::min({ngr[i], kMaxRunKeys / P.gran[i], qasr::kDecodeMaxRunGranules}));
        keys += (int64_t)nkvh * P.len[i];
        pairs += nkvh;
    }
    const bool split = env_int("QASR_DECODE_SPLIT", 1) != 0;  // 0: every (entry, kv head) whole
    if (!split) {
        // runs as long as a workgroup's LDS allows (kDecodeMaxRunGranules)
    } else if (pairs < target) {
        auto runs_for = [&](int64_t c, int i) {
            return (int)std::max<int64_t>(1, std::min<int64_t>(run[i], c / P.gran[i]));
        };
        auto wgs_for = [&](int64_t c) {
            int64_t t = 0;
            for (int i = 0; i < P.batch; ++i) t += (int64_t)nkvh * ceil_div(ngr[i], runs_for(c, i));
            return t;
        };
        int64_t c = qasr::kDecodeGranuleQuantum;
        int64_t cmax = 0;
        for (int i = 0; i < P.batch; ++i) cmax = std::max<int64_t>(cmax, (int64_t)ngr[i] * P.gran[i]);
        while (c < cmax && wgs_for(c) > target) c += qasr::kDecodeGranuleQuantum;
        for (int i = 0; i < P.batch; ++i) run[i] = runs_for(c, i);
    } else {
        int wgs = 0;
        for (int i = 0; i < P.batch; ++i) wgs += nkvh * ceil_div(ngr[i], run[i]);
        const int max_wgs = 4 * std::max(target, pairs);
        auto run_keys = [&](int i) { return std::min<int64_t>((int64_t)run[i] * P.gran[i], P.len[i]); };
        while (wgs + nkvh <= max_wgs) {
            int best = -1;
            int64_t best_keys = 0;
            for (int i = 0; i < P.batch; ++i)
                if (run[i] > 1 && run_keys(i) > best_keys) {
                    best = i;
                    best_keys = run_keys(i);
                }
            if (best < 0 || 2 * best_keys * wgs <= 3 * keys) break;
            const int nw = ceil_div(ngr[best], run[best]);
            const int r = std::min(run[best] - 1, ceil_div(ngr[best], nw + 1));  // run shrinks every time
            wgs += nkvh * (ceil_div(ngr[best], r) - nw);
            run[best] = r;
        }
    }
    P.wg_base[0] = 0;
    P.part_base[0] = 0;
    for (int i = 0; i < P.batch; ++i) {
        P.run[i] = run[i];
        P.wg_base[i + 1] = P.wg_base[i] + nkvh * ceil_div(ngr[i], run[i]);
        P.part_base[i + 1] = P.part_base[i] + nkvh * ngr[i];
    }
}

int check_common(qasr_ctx* ctx, qasr_kv* kv, int layer) {
    if (!ctx || !kv) return fail(QASR_EINVAL, "null context or KV pool");
    if (kv->ctx != ctx) return fail(QASR_EINVAL, "KV pool belongs to another context");
    if (layer < 0 || layer >= ctx->cfg.num_hidden_layers)
        return fail(QASR_EINVAL, "layer %d outside [0, %d)", layer, ctx->cfg.num_hidden_layers);
    return QASR_OK;
}

int run_decode(bool fused, qasr_ctx* ctx, qasr_kv* kv, int layer, int batch, const int32_t* slots,
               const int32_t* lens, const void* qin, const void* q_gain, const void* k_gain,
               void* out, void* stream) {
    const qasr_attn_cfg& c = ctx->cfg;
    const int nqh = c.num_attention_heads, nkvh = c.num_key_value_heads;
    const int64_t in_row = fused ? (int64_t)(nqh + 2 * nkvh) * qasr::kHeadDim
                                 : (int64_t)nqh * qasr::kHeadDim;
    const int64_t out_row = (int64_t)nqh * qasr::kHeadDim;
    const qasr::CacheGeom g = geom(kv);
    qasr::DecodeWs ws{kv->dws_acc, kv->dws_ml, kv->dws_ctr, kv->dws_items};
    for (int b0 = 0; b0 < batch; b0 += qasr::kMaxBatch) {
        const int nb = std::min(qasr::kMaxBatch, batch - b0);
        qasr::DecodePlan P{};
        P.batch = nb;
        P.nqh = nqh;
        P.eps = c.rms_norm_eps;
        P.scale_log2 = ctx->scale_log2;
        for (int i = 0; i < nb; ++i) {
            P.slot[i] = slots ? slots[b0 + i] : b0 + i;
            P.len[i] = lens[b0 + i];
        }
        plan_decode_granules(P, nkvh, ctx->cus);
        const f16* qp = (const f16*)qin + b0 * in_row;
        f16* op = (f16*)out + b0 * out_row;
        hipError_t e = qasr::launch_decode_attn(fused, g, layer, P, P.wg_base[nb], qp,
                                                (const f16*)q_gain, (const f16*)k_gain, ctx->cos,
                                                ctx->sin, op, ws, (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "decode attention launch");
    }
    return QASR_OK;
}

// ---- prefill: planning shared by every prefill entry point ----------------

// Split workspace of qasr_prefill_attn_noalloc, for callers that cannot
// allocate (HIP graph capture, serving loops, harnesses that forbid it): a
// file-scope device array, one copy per GPU, alive until the process ends.
// Partials of at most kScratchItems work items (34 MB) plus the arrival
// counters.  Host code reaches it only through the address resolved per
// device by hipGetSymbolAddress (scratch_ptr); the array's name is a host
// stand-in, not a device address.
constexpr int64_t kScratchItems = 512;
constexpr int kScratchMaxKvHeads = 16;  // nkvh <= 16 (qasr_ctx_create's head limit)
constexpr int64_t kScratchO = kScratchItems * qasr::kPrefillItemFloats;
constexpr int64_t kScratchMl = kScratchItems * qasr::kPrefillItemMl;
constexpr int64_t kScratchCounters = (int64_t)kScratchMaxKvHeads * qasr::kMaxLaunchRowBlocks;
static __device__ __align__(256) float scratch[kScratchO + kScratchMl + kScratchCounters];

constexpr int kMaxDevices = 64;
// Key ranges of up to 1024 keys run unsplit, in 32-row blocks.  Measured
// per layer, against 64-row blocks with key splits: 640 rows from 0 12.5
// against 16.1 us, 1024 from 0 16.6 against 18.6, 256 at 512 13.0 against
// 15.9, 64 at 960 15.6 against 15.5; past 1024 keys the splits win (2048
// rows from 0: 37.3 against 39.3 us unsplit in 32-row blocks).
constexpr int kPrefillNoSplitTiles = 8;
std::mutex g_scratch_mu;
float* g_scratch_dev[kMaxDevices] = {};

// Device address of `scratch` on `device` (resolved once per device, with
// that device current).
int scratch_ptr(int device, float** out) {
    if (device < 0 || device >= kMaxDevices) return fail(QASR_EINVAL, "device %d beyond %d", device, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[device]) {
        DeviceScope ds(device);
        if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
        void* p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        if (!p) return fail(QASR_EDEVICE, "no device address for the prefill scratch array");
        g_scratch_dev[device] = (float*)p;
    }
    *out = g_scratch_dev[device];
    return QASR_OK;
}

__global__ void zero_u32_kernel(uint32_t* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Longest prefill one qasr_prefill_attn_noalloc call takes.  A default plan
// of r rows has at most 256 + nkvh * ceil(r / 64) work items: a split plan
// at most 256, an unsplit 16-row one too, an unsplit 64-row one
// nkvh * ceil(r / 64), an unsplit 32-row one (key ranges of at most 1024
// keys, so r <= 1024) nkvh * ceil(r / 32) <= 2 nkvh * ceil(r / 64) <= 256 +
// nkvh * ceil(r / 64) for nkvh <= 16.  Up to
// this many rows every default plan fits the scratch array, and the
// no-allocation call runs exactly qasr_prefill_attn's items.
int noalloc_max_rows(int nkvh) {
    const int64_t rbs = std::min<int64_t>(qasr::kMaxRowBlocks, (kScratchItems - 256) / nkvh);
    return qasr::kPrefillRows * (int)rbs;
}

// The plan of one piece of `rows` (<= kMaxRowBlocks * kPrefillRows) rows at
// kv_start `ks`, a function of (rows, ks, nkvh) alone.  Tiles per split: the
// fewest that keep the work items within one workgroup per CU for 256 CUs
// (every row block rounds its split count up, so that is checked row block
// by row block); when even unsplit row blocks are more, none is split.  A
// few items past 256 wait for a whole second round: 1500 rows at 2000, 304
// items at 21 tiles per split, 81.5 us per layer, against 57.6 us for 256
// items at 24.  A split's merge (publish, ticket, read back) is about three
// memory round trips, as long as several latency-bound tiles: key ranges of
// up to kPrefillNoSplitTiles tiles are never split.  Unsplit short ranges
// also take 16-row blocks when their items fit 256, else 32-row blocks:
// more workgroups, less work on the longest one.  A forced split count (tps_forced > 0, QASR_PREFILL_TPS)
// keeps 64-row blocks.
qasr::PrefillPlan choose_prefill_plan(int rows, int ks, int nkvh, int tps_forced) {
    const int nrb = (rows + qasr::kPrefillRows - 1) / qasr::kPrefillRows;
    const int max_tiles = (ks + rows + qasr::kPrefillTileKeys - 1) / qasr::kPrefillTileKeys;
    int tps = tps_forced;
    int rb_rows = qasr::kPrefillRows;
    if (tps <= 0) {
        const int64_t want = std::max<int64_t>(1, 256 / nkvh);  // items per kv head
        if (max_tiles <= kPrefillNoSplitTiles) {
            // Unsplit: 16-row blocks (one wave per SIMD, both q heads in its
            // MFMA columns) while their items fit one workgroup per CU for
            // 256 CUs, else 32-row blocks.
            tps = max_tiles;
            const int64_t nrb16 = (rows + qasr::kPrefillRows / 4 - 1) / (qasr::kPrefillRows / 4);
            rb_rows = nrb16 <= qasr::kMaxRowBlocks && nrb16 * nkvh <= 256 ? qasr::kPrefillRows / 4
                                                                          : qasr::kPrefillRows / 2;
        } else {
            // Items at t tiles per split: sum over row blocks of ceil(tiles / t),
            // at least sum(tiles) / t, so t starts at sum(tiles) / want.
            auto row_tiles = [&](int rb) {
                const int kend = ks + std::min((rb + 1) * qasr::kPrefillRows, rows);
                return (kend + qasr::kPrefillTileKeys - 1) / qasr::kPrefillTileKeys;
            };
            int64_t sum = 0;
            for (int rb = 0; rb < nrb; ++rb) sum += row_tiles(rb);
            tps = max_tiles;
            for (int t = (int)std::max<int64_t>(2, (sum + want - 1) / want); t < max_tiles; ++t) {
                int64_t n = 0;
                for (int rb = 0; rb < nrb; ++rb) n += (row_tiles(rb) + t - 1) / t;
                if (n <= want) {
                    tps = t;
                    break;
                }
            }
        }
    }
    return qasr::plan_prefill(rows, ks, nkvh, tps, rb_rows);
}

// One piece: up to kMaxRowBlocks * kPrefillRows rows of one segment.
struct Piece {
    int slot, ks, rows;
    int64_t row_base;
    qasr::PrefillPlan P;
};

// One launch: pieces [first, first + n) of a list, all of one row block size.
struct PrefillLaunch {
    qasr::PrefillSegs S;
    int rows_per_block;
    int64_t records;
};

// Causal prefill attention of nseg segments (rows concatenated in segment
// order in q / out).  Every segment is cut into pieces of at most 4096 rows
// and every piece planned by choose_prefill_plan, so a segment runs the same
// work items (and so gets the same bits) whether it comes alone or with
// others.  Pieces of one row block size are packed into launches of at most
// kMaxPrefillPieces pieces, kMaxLaunchRowBlocks row blocks and `cap` partial
// records.  Every check runs before the first launch.
int run_prefill_segments(qasr_ctx* ctx, qasr_kv* kv, int layer, const qasr_segment* segs,
                         int nseg, const void* q_dev, void* out_dev, void* stream, bool noalloc) {
    int rc = check_common(ctx, kv, layer);
    if (rc) return rc;
    if (nseg < 0 || (nseg > 0 && !segs)) return fail(QASR_EINVAL, "bad segment list");
    const qasr_attn_cfg& c = ctx->cfg;
    const int nqh = c.num_attention_heads, nkvh = c.num_key_value_heads;
    int64_t total = 0;
    for (int i = 0; i < nseg; ++i) {
        const qasr_segment& g = segs[i];
        if (g.slot < 0 || g.slot >= kv->slots)
            return fail(QASR_EINVAL, "segment %d: slot %d outside [0, %d)", i, g.slot, kv->slots);
        if (g.pos0 < 0 || g.rows < 0) return fail(QASR_EINVAL, "segment %d: negative kv_start/rows", i);
        const int64_t end = (int64_t)g.pos0 + g.rows;
        if (end > c.max_seq)
            return fail(QASR_ERANGE, "segment %d: prefill needs %lld positions, max_seq is %d", i,
                        (long long)end, c.max_seq);
        if (end > kv->cap)
            return fail(QASR_ERANGE, "segment %d: prefill needs %lld positions, KV capacity is %d",
                        i, (long long)end, kv->cap);
        total += g.rows;
    }
    if (total == 0) return QASR_OK;
    if (!q_dev || !out_dev) return fail(QASR_EINVAL, "null device pointer");
    if (noalloc) {
        if (nkvh > kScratchMaxKvHeads)
            return fail(QASR_EINVAL, "%d kv heads: the no-allocation prefill takes at most %d",
                        nkvh, kScratchMaxKvHeads);
        if (total > noalloc_max_rows(nkvh))
            return fail(QASR_EINVAL, "%lld rows: the no-allocation prefill takes at most %d rows per "
                        "call (prefill longer prompts in chunks, kv_start > 0)", (long long)total,
                        noalloc_max_rows(nkvh));
        if (!ctx->scratch) return fail(QASR_ESTATE, "context has no prefill scratch address");
    }
    const int tps_forced = env_int("QASR_PREFILL_TPS", 0);
    const int piece_rows = qasr::kMaxRowBlocks * qasr::kPrefillRows;
    std::vector<Piece> pieces;
    int64_t r0 = 0;
    for (int i = 0; i < nseg; ++i) {
        for (int p0 = 0; p0 < segs[i].rows; p0 += piece_rows) {
            Piece pc;
            pc.slot = segs[i].slot;
            pc.ks = segs[i].pos0 + p0;
            pc.rows = std::min(piece_rows, segs[i].rows - p0);
            pc.row_base = r0 + p0;
            pc.P = choose_prefill_plan(pc.rows, pc.ks, nkvh, tps_forced);
            pieces.push_back(pc);
        }
        r0 += segs[i].rows;
    }
    // Many short pieces in one launch (the batched prefill): their 16-row
    // blocks would make several rounds of one-wave-per-SIMD workgroups, so
    // they run as 32-row blocks (eight waves) instead.  Both kernels give
    // every row the same bits: the same MFMAs per output column, the same
    // four 32-key groups combined in the same order, masks and rescales per
    // lane, and a skipped all-masked half tile only adds zeros.  So a
    // segment's output still does not depend on its batch mates.
    {
        int64_t items16 = 0;
        for (const Piece& pc : pieces)
            if (pc.P.rows_per_block == qasr::kPrefillRows / 4) items16 += (int64_t)nkvh * pc.P.items_per_kvh;
        if (items16 > 256)
            for (Piece& pc : pieces)
                if (pc.P.rows_per_block == qasr::kPrefillRows / 4)
                    pc.P = qasr::plan_prefill(pc.rows, pc.ks, nkvh, pc.P.tps, qasr::kPrefillRows / 2);
    }
    const qasr::CacheGeom g = geom(kv);
    const int64_t cap = noalloc ? kScratchItems : std::numeric_limits<int64_t>::max();
    std::vector<PrefillLaunch> launches;
    for (const int rpb : {qasr::kPrefillRows, qasr::kPrefillRows / 2, qasr::kPrefillRows / 4}) {
        PrefillLaunch* L = nullptr;
        for (const Piece& pc : pieces) {
            if (pc.P.rows_per_block != rpb) continue;
            const int64_t recs = (int64_t)nkvh * pc.P.items_per_kvh;
            if (recs > cap)
                return fail(QASR_EINVAL, "prefill plan of %lld items exceeds the scratch's %lld",
                            (long long)recs, (long long)cap);
            if (L) {
                const qasr::PrefillSegs& S = L->S;
                const int rbs = S.rb_base[S.n - 1] + S.nrb[S.n - 1];
                if (S.n == qasr::kMaxPrefillPieces || rbs + pc.P.nrb > qasr::kMaxLaunchRowBlocks ||
                    L->records + recs > cap)
                    L = nullptr;
            }
            if (!L) {
                launches.emplace_back();
                L = &launches.back();
                std::memset(&L->S, 0, sizeof L->S);
                L->rows_per_block = rpb;
                L->records = 0;
            }
            qasr::PrefillSegs& S = L->S;
            const int i = S.n;
            const int rb0 = i ? S.rb_base[i - 1] + S.nrb[i - 1] : 0;
            S.rb_base[i] = rb0;
            S.nrb[i] = pc.P.nrb;
            S.tps[i] = pc.P.tps;
            S.kv_start[i] = pc.ks;
            S.rows[i] = pc.rows;
            S.row_base[i] = (int32_t)pc.row_base;
            S.kv_off[i] = (int64_t)pc.slot * g.slot_stride + (int64_t)layer * g.layer_stride;
            S.part_base[i] = (int32_t)L->records;
            for (int rb = 0; rb <= pc.P.nrb; ++rb) S.sp[rb0 + i + rb] = pc.P.sp_base[rb];
            S.item_base[i + 1] = S.item_base[i] + (int32_t)recs;
            S.n = i + 1;
            L->records += recs;
        }
    }
    if (total > INT32_MAX / (nqh * qasr::kHeadDim))
        return fail(QASR_EINVAL, "%lld prefill rows exceed the row index range", (long long)total);
    int64_t need = 0;
    for (const PrefillLaunch& L : launches) need = std::max(need, L.records);
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    qasr::PrefillWs ws{};
    if (noalloc) {
        ws.o = ctx->scratch;
        ws.ml = ctx->scratch + kScratchO;
        ws.counters = reinterpret_cast<uint32_t*>(ctx->scratch + kScratchO + kScratchMl);
        ws.items = kScratchItems;
    } else {
        rc = ensure_prefill_ws(kv, need);
        if (rc) return rc;
        ws = qasr::PrefillWs{kv->pws_o, kv->pws_ml, kv->pws_ctr, kv->pws_items};
    }
    if (noalloc) {
        // The array keeps the last call's contents: the arrival counters
        // start this call at zero.
        const int n = nkvh * qasr::kMaxLaunchRowBlocks;
        hipLaunchKernelGGL(zero_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                           ws.counters, n);
        HIP_TRY(hipGetLastError(), "scratch counter clear");
    }
    qasr::PrefillArgs a;
    a.q = (const f16*)q_dev;
    a.out = (f16*)out_dev;
    a.k = g.base;
    a.v = g.base + g.kv_stride;
    a.head_stride = g.head_stride;
    a.nqh = nqh;
    a.nkvh = nkvh;
    a.s = 0;
    a.kv_start = 0;
    a.scale_log2 = ctx->scale_log2;
    for (const PrefillLaunch& L : launches) {
        const hipError_t e = qasr::launch_prefill_attn(a, L.rows_per_block, L.S, ws, (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "prefill attention launch");
    }
    return QASR_OK;
}

}  // namespace

extern "C" {

int qasr_abi_version(void) { return QASR_ABI_VERSION; }

const char* qasr_last_error(void) { return g_err.c_str(); }

int qasr_ctx_create(const qasr_attn_cfg* cfg, int device, qasr_ctx** out) {
    if (!cfg || !out) return fail(QASR_EINVAL, "null argument");
    *out = nullptr;
    const qasr_attn_cfg& c = *cfg;
    if (c.head_dim != qasr::kHeadDim)
        return fail(QASR_EINVAL, "head_dim %d unsupported (this build is specialised for 128)",
                    c.head_dim);
    if (c.num_key_value_heads <= 0 || c.num_attention_heads != qasr::kRep * c.num_key_value_heads)
        return fail(QASR_EINVAL, "%d q heads / %d kv heads: the kernels need exactly 2 q heads per "
                    "kv head", c.num_attention_heads, c.num_key_value_heads);
    if (c.num_attention_heads + c.num_key_value_heads > 48)
        return fail(QASR_EINVAL, "too many heads (%d + %d)", c.num_attention_heads,
                    c.num_key_value_heads);
    if (c.num_hidden_layers <= 0) return fail(QASR_EINVAL, "num_hidden_layers must be > 0");
    if (c.max_seq <= 0 || c.max_seq > kMaxPositions)
        return fail(QASR_EINVAL, "max_seq %d outside [1, %d]", c.max_seq, kMaxPositions);
    if (!(c.rms_norm_eps >= 0.0f) || !std::isfinite(c.rms_norm_eps))
        return fail(QASR_EINVAL, "rms_norm_eps must be finite and >= 0");
    int ndev = 0;
    HIP_TRY(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
    if (device < 0 || device >= ndev)
        return fail(QASR_EINVAL, "device %d outside [0, %d)", device, ndev);
    int cus = 0;
    HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
            "hipDeviceGetAttribute");
    float* scratch_dev = nullptr;
    int src = scratch_ptr(device, &scratch_dev);
    if (src != QASR_OK) return src;
    qasr_ctx* ctx = new qasr_ctx();
    ctx->cfg = c;
    ctx->device = device;
    ctx->scratch = scratch_dev;
    ctx->cus = std::max(1, cus);
    // scale = 1/sqrt(hd) in f32 (decoder.rs:204-206), folded with log2(e) so the
    // kernels exponentiate with exp2.
    const float scale = 1.0f / std::sqrt((float)c.head_dim);
    ctx->scale_log2 = (float)((double)scale * 1.4426950408889634073599246810019);
    *out = ctx;
    return QASR_OK;
}

void qasr_ctx_destroy(qasr_ctx* ctx) {
    if (!ctx) return;
    DeviceScope ds(ctx->device);
    (void)hipDeviceSynchronize();  // no launch in flight still reads the tables
    if (ctx->cos) (void)hipFree(ctx->cos);
    if (ctx->sin) (void)hipFree(ctx->sin);
    delete ctx;
}

int qasr_mrope_text_tables(int rows, int head_dim, double rope_theta,
                           const int32_t* mrope_section, int nsec, int interleaved,
                           uint16_t* cos_f16, uint16_t* sin_f16) {
    if (rows < 0 || head_dim <= 0 || head_dim % 2 || !cos_f16 || !sin_f16 || !mrope_section ||
        nsec <= 0)
        return fail(QASR_EINVAL, "bad table arguments");
    const int half = head_dim / 2;
    // build_dim_map (mrope.rs:5-41): axis per frequency.
    std::vector<int> dm;
    if (interleaved) {
        std::vector<int> used(nsec, 0);
        while ((int)dm.size() < half) {
            const size_t before = dm.size();
            for (int d = 0; d < nsec && (int)dm.size() < half; ++d)
                if (used[d] < mrope_section[d]) {
                    dm.push_back(d);
                    ++used[d];
                }
            if (dm.size() == before) break;
        }
    } else {
        for (int d = 0; d < nsec; ++d)
            for (int i = 0; i < mrope_section[d] && (int)dm.size() < half; ++i) dm.push_back(d);
        while ((int)dm.size() < half) dm.push_back(nsec - 1);
    }
    if ((int)dm.size() != half) return fail(QASR_EINVAL, "mrope_section quotas cover fewer than %d "
                                            "frequencies", half);
    for (int d : dm)
        if (d > 2) return fail(QASR_EINVAL, "mrope_section has more than 3 axes");
    // Text positions put the same t on all three axes (mrope.rs:77-80), so
    // angle = t * theta^(-2j/hd) whatever the axis map; f64 -> f32 -> f16 RNE
    // (mrope.rs:55-71, inference.rs:1046-1047).
    std::vector<double> inv(half);
    for (int j = 0; j < half; ++j) inv[j] = 1.0 / std::pow(rope_theta, 2.0 * j / (double)head_dim);
    for (int t = 0; t < rows; ++t) {
        for (int j = 0; j < half; ++j) {
            const double angle = (double)t * inv[j];
            const uint16_t cb = f16_bits((float)std::cos(angle));
            const uint16_t sb = f16_bits((float)std::sin(angle));
            const int64_t o = (int64_t)t * head_dim + j;
            cos_f16[o] = cos_f16[o + half] = cb;
            sin_f16[o] = sin_f16[o + half] = sb;
        }
    }
    return QASR_OK;
}

int qasr_set_rope_tables(qasr_ctx* ctx, const uint16_t* cos_f16, const uint16_t* sin_f16,
                         int rows) {
    if (!ctx || !cos_f16 || !sin_f16 || rows <= 0) return fail(QASR_EINVAL, "bad table arguments");
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    const size_t bytes = (size_t)rows * ctx->cfg.head_dim * sizeof(uint16_t);
    HIP_TRY(hipDeviceSynchronize(), "rope tables sync");  // no launch in flight reads the old ones
    if (ctx->cos) (void)hipFree(ctx->cos);
    if (ctx->sin) (void)hipFree(ctx->sin);
    ctx->cos = ctx->sin = nullptr;
    ctx->rope_rows = 0;
    HIP_TRY(hipMalloc(&ctx->cos, bytes), "rope tables");
    HIP_TRY(hipMalloc(&ctx->sin, bytes), "rope tables");
    HIP_TRY(hipMemcpy(ctx->cos, cos_f16, bytes, hipMemcpyHostToDevice), "rope upload");
    HIP_TRY(hipMemcpy(ctx->sin, sin_f16, bytes, hipMemcpyHostToDevice), "rope upload");
    ctx->rope_rows = rows;
    return QASR_OK;
}

int qasr_kv_create(qasr_ctx* ctx, int slots, int cap, qasr_kv** out) {
    if (!ctx || !out) return fail(QASR_EINVAL, "null argument");
    *out = nullptr;
    if (slots <= 0) return fail(QASR_EINVAL, "slots must be > 0");
    if (cap <= 0) return fail(QASR_EINVAL, "cap must be > 0");
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    qasr_kv* kv = new qasr_kv();
    kv->ctx = ctx;
    kv->slots = slots;
    kv->cap = target_cap(cap, 0, ctx->cfg.max_seq);
    const qasr::CacheGeom g = geom(kv);
    kv->bytes = (size_t)g.slot_stride * slots * sizeof(f16);
    hipError_t e = hipMalloc(&kv->base, kv->bytes);
    if (e == hipSuccess) e = hipMemset(kv->base, 0, kv->bytes);
    if (e != hipSuccess) {
        if (kv->base) (void)hipFree(kv->base);
        delete kv;
        return hip_fail(e, "KV pool allocation");
    }
    int rc = alloc_decode_ws(kv);
    if (rc != QASR_OK) {
        qasr_kv_destroy(kv);
        return rc;
    }
    *out = kv;
    return QASR_OK;
}

void qasr_kv_destroy(qasr_kv* kv) {
    if (!kv) return;
    DeviceScope ds(kv->ctx->device);
    (void)hipDeviceSynchronize();
    if (kv->base) (void)hipFree(kv->base);
    free_decode_ws(kv);
    free_prefill_ws(kv);
    delete kv;
}

int qasr_kv_get_info(const qasr_kv* kv, qasr_kv_info* out) {
    if (!kv || !out) return fail(QASR_EINVAL, "null argument");
    const qasr::CacheGeom g = geom(kv);
    out->base_dev = kv->base;
    out->slots = kv->slots;
    out->layers = kv->ctx->cfg.num_hidden_layers;
    out->nkvh = g.nkvh;
    out->cap = kv->cap;
    out->head_dim = qasr::kHeadDim;
    out->slot_stride = g.slot_stride;
    out->layer_stride = g.layer_stride;
    out->kv_stride = g.kv_stride;
    out->head_stride = g.head_stride;
    out->bytes = kv->bytes;
    return QASR_OK;
}

int qasr_kv_ensure_capacity(qasr_kv* kv, int need, int keep_rows, int* cap_out) {
    if (!kv) return fail(QASR_EINVAL, "null KV pool");
    if (need < 0 || keep_rows < 0) return fail(QASR_EINVAL, "negative need / keep_rows");
    const int target = target_cap(need, kv->cap, kv->ctx->cfg.max_seq);
    if (target == kv->cap) {
        if (cap_out) *cap_out = kv->cap;
        return QASR_OK;
    }
    DeviceScope ds(kv->ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    const int prev = kv->cap;
    const qasr::CacheGeom og = geom(kv);
    qasr_kv tmp = *kv;
    tmp.cap = target;
    const qasr::CacheGeom ng = geom(&tmp);
    const size_t nbytes = (size_t)ng.slot_stride * kv->slots * sizeof(f16);
    // Work queued on any stream (a step still appending row pos-1 on a
    // non-blocking stream, say) completes before the rows are copied: the
    // copy below runs on the null stream, which does not order non-blocking
    // streams.
    HIP_TRY(hipDeviceSynchronize(), "KV pool growth sync");
    f16* nb = nullptr;
    HIP_TRY(hipMalloc(&nb, nbytes), "KV pool growth");
    hipError_t e = hipMemset(nb, 0, nbytes);
    // Keep rows 0..keep_rows-1 of every (slot, layer, K/V, head): one pitched
    // copy, as the reference copies each head's prefix (decoder.rs:1617-1650).
    const int rows = std::min(keep_rows, prev);
    if (e == hipSuccess && rows > 0) {
        const size_t height = (size_t)kv->slots * kv->ctx->cfg.num_hidden_layers * 2 * og.nkvh;
        e = hipMemcpy2D(nb, (size_t)ng.head_stride * sizeof(f16), kv->base,
                        (size_t)og.head_stride * sizeof(f16),
                        (size_t)rows * qasr::kHeadDim * sizeof(f16), height,
                        hipMemcpyDeviceToDevice);
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        (void)hipFree(nb);
        return hip_fail(e, "KV pool growth copy");
    }
    (void)hipFree(kv->base);
    kv->base = nb;
    kv->bytes = nbytes;
    kv->cap = target;
    free_decode_ws(kv);
    int rc = alloc_decode_ws(kv);
    if (rc != QASR_OK) return rc;
    if (cap_out) *cap_out = kv->cap;
    return QASR_OK;
}

int qasr_qk_norm_rope_append(qasr_ctx* ctx, qasr_kv* kv, int layer, const qasr_segment* segs,
                             int nseg, const void* qkv_dev, const void* q_gain_dev,
                             const void* k_gain_dev, void* q_out_dev, void* stream) {
    int rc = check_common(ctx, kv, layer);
    if (rc) return rc;
    if (nseg < 0 || (nseg > 0 && !segs)) return fail(QASR_EINVAL, "bad segment list");
    if (nseg == 0) return QASR_OK;
    if (!qkv_dev || !q_gain_dev || !k_gain_dev || !q_out_dev)
        return fail(QASR_EINVAL, "null device pointer");
    if (!ctx->cos) return fail(QASR_ESTATE, "RoPE tables not set (qasr_set_rope_tables)");
    for (int i = 0; i < nseg; ++i) {
        const qasr_segment& s = segs[i];
        if (s.slot < 0 || s.slot >= kv->slots)
            return fail(QASR_EINVAL, "segment %d: slot %d outside [0, %d)", i, s.slot, kv->slots);
        if (s.pos0 < 0 || s.rows < 0) return fail(QASR_EINVAL, "segment %d: negative pos/rows", i);
        const int64_t end = (int64_t)s.pos0 + s.rows;
        if (end > kv->cap)
            return fail(QASR_ERANGE, "segment %d: positions up to %lld exceed KV capacity %d", i,
                        (long long)end, kv->cap);
        if (end > ctx->cfg.max_seq)
            return fail(QASR_ERANGE, "segment %d: %lld positions exceed max_seq %d", i,
                        (long long)end, ctx->cfg.max_seq);
        if (end > ctx->rope_rows)
            return fail(QASR_ERANGE, "segment %d: positions beyond the %d RoPE table rows", i,
                        ctx->rope_rows);
    }
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    const qasr_attn_cfg& c = ctx->cfg;
    const int64_t in_row = (int64_t)(c.num_attention_heads + 2 * c.num_key_value_heads) * 128;
    const int64_t q_row = (int64_t)c.num_attention_heads * 128;
    const qasr::CacheGeom g = geom(kv);
    int64_t row_off = 0;
    for (int s0 = 0; s0 < nseg; s0 += qasr::kMaxBatch) {
        const int ns = std::min(qasr::kMaxBatch, nseg - s0);
        qasr::SegPlan P{};
        P.nseg = ns;
        P.nqh = c.num_attention_heads;
        P.eps = c.rms_norm_eps;
        P.row_base[0] = 0;
        for (int i = 0; i < ns; ++i) {
            P.slot[i] = segs[s0 + i].slot;
            P.pos0[i] = segs[s0 + i].pos0;
            P.row_base[i + 1] = P.row_base[i] + segs[s0 + i].rows;
        }
        hipError_t e = qasr::launch_norm_rope_append(
            g, layer, P, (const f16*)qkv_dev + row_off * in_row, (const f16*)q_gain_dev,
            (const f16*)k_gain_dev, ctx->cos, ctx->sin, (f16*)q_out_dev + row_off * q_row,
            (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "stage (a) launch");
        row_off += P.row_base[ns];
    }
    return QASR_OK;
}

static int check_batch(qasr_ctx* ctx, qasr_kv* kv, int batch, const int32_t* slots,
                       bool distinct) {
    if (batch < 0) return fail(QASR_EINVAL, "negative batch");
    if (batch > kv->slots && distinct)
        return fail(QASR_EINVAL, "batch %d larger than the pool's %d slots", batch, kv->slots);
    if (slots) {
        std::vector<char> seen(kv->slots, 0);
        for (int b = 0; b < batch; ++b) {
            if (slots[b] < 0 || slots[b] >= kv->slots)
                return fail(QASR_EINVAL, "entry %d: slot %d outside [0, %d)", b, slots[b],
                            kv->slots);
            if (distinct && seen[slots[b]]++)
                return fail(QASR_EINVAL, "entry %d: slot %d appears twice", b, slots[b]);
        }
    } else if (batch > kv->slots) {
        return fail(QASR_EINVAL, "batch %d larger than the pool's %d slots", batch, kv->slots);
    }
    (void)ctx;
    return QASR_OK;
}

int qasr_decode_attn(qasr_ctx* ctx, qasr_kv* kv, int layer, int batch, const int32_t* slots,
                     const int32_t* cur_len, const void* q_dev, void* out_dev, void* stream) {
    int rc = check_common(ctx, kv, layer);
    if (rc) return rc;
    rc = check_batch(ctx, kv, batch, slots, false);
    if (rc) return rc;
    if (batch == 0) return QASR_OK;
    if (!cur_len || !q_dev || !out_dev) return fail(QASR_EINVAL, "null argument");
    for (int b = 0; b < batch; ++b) {
        if (cur_len[b] <= 0) return fail(QASR_EINVAL, "entry %d: cur_len %d must be > 0", b, cur_len[b]);
        if (cur_len[b] > kv->cap)
            return fail(QASR_ERANGE, "entry %d: cur_len %d exceeds KV capacity %d", b, cur_len[b],
                        kv->cap);
        if (cur_len[b] > ctx->cfg.max_seq)
            return fail(QASR_ERANGE, "entry %d: cur_len %d exceeds max_seq %d", b, cur_len[b],
                        ctx->cfg.max_seq);
    }
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    return run_decode(false, ctx, kv, layer, batch, slots, cur_len, q_dev, nullptr, nullptr, out_dev,
                      stream);
}

int qasr_decode_step(qasr_ctx* ctx, qasr_kv* kv, int layer, int batch, const int32_t* slots,
                     const int32_t* pos, const void* qkv_dev, const void* q_gain_dev,
                     const void* k_gain_dev, void* out_dev, void* stream) {
    int rc = check_common(ctx, kv, layer);
    if (rc) return rc;
    rc = check_batch(ctx, kv, batch, slots, true);
    if (rc) return rc;
    if (batch == 0) return QASR_OK;
    if (!pos || !qkv_dev || !q_gain_dev || !k_gain_dev || !out_dev)
        return fail(QASR_EINVAL, "null argument");
    if (!ctx->cos) return fail(QASR_ESTATE, "RoPE tables not set (qasr_set_rope_tables)");
    std::vector<int32_t> lens(batch);
    for (int b = 0; b < batch; ++b) {
        if (pos[b] < 0) return fail(QASR_EINVAL, "entry %d: negative position", b);
        if (pos[b] >= kv->cap)
            return fail(QASR_ERANGE, "entry %d: position %d beyond KV capacity %d", b, pos[b],
                        kv->cap);
        if (pos[b] >= ctx->cfg.max_seq)
            return fail(QASR_ERANGE, "entry %d: decode past max_seq %d", b, ctx->cfg.max_seq);
        if (pos[b] >= ctx->rope_rows)
            return fail(QASR_ERANGE, "entry %d: position %d beyond the %d RoPE table rows", b,
                        pos[b], ctx->rope_rows);
        lens[b] = pos[b] + 1;
    }
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    return run_decode(true, ctx, kv, layer, batch, slots, lens.data(), qkv_dev, q_gain_dev,
                      k_gain_dev, out_dev, stream);
}

int qasr_prefill_attn(qasr_ctx* ctx, qasr_kv* kv, int layer, int slot, int kv_start, int s,
                      const void* q_dev, void* out_dev, void* stream) {
    const qasr_segment seg{slot, kv_start, s};
    return run_prefill_segments(ctx, kv, layer, &seg, 1, q_dev, out_dev, stream, false);
}

int qasr_prefill_attn_noalloc(qasr_ctx* ctx, qasr_kv* kv, int layer, int slot, int kv_start,
                              int s, const void* q_dev, void* out_dev, void* stream) {
    const qasr_segment seg{slot, kv_start, s};
    return run_prefill_segments(ctx, kv, layer, &seg, 1, q_dev, out_dev, stream, true);
}

int qasr_prefill_attn_batch(qasr_ctx* ctx, qasr_kv* kv, int layer, const qasr_segment* segs,
                            int nseg, const void* q_dev, void* out_dev, void* stream) {
    return run_prefill_segments(ctx, kv, layer, segs, nseg, q_dev, out_dev, stream, false);
}

int qasr_plan_decode(int batch, const int32_t* lens, int nkvh, int cus, int32_t* gran_out,
                     int32_t* run_out, int32_t* wg_base_out) {
    if (batch < 1 || batch > qasr::kMaxBatch)
        return fail(QASR_EINVAL, "batch %d outside [1, %d]", batch, qasr::kMaxBatch);
    if (nkvh < 1 || nkvh > 64 || cus < 1) return fail(QASR_EINVAL, "nkvh %d / cus %d", nkvh, cus);
    if (!lens || !gran_out || !run_out || !wg_base_out) return fail(QASR_EINVAL, "null pointer");
    qasr::DecodePlan P{};
    P.batch = batch;
    for (int b = 0; b < batch; ++b) {
        if (lens[b] < 1 || lens[b] > kMaxPositions)
            return fail(QASR_EINVAL, "entry %d attends %d keys (at most %d)", b, lens[b], kMaxPositions);
        P.len[b] = lens[b];
    }
    plan_decode_granules(P, nkvh, cus);
    for (int b = 0; b < batch; ++b) {
        gran_out[b] = P.gran[b];
        run_out[b] = P.run[b];
    }
    for (int b = 0; b <= batch; ++b) wg_base_out[b] = P.wg_base[b];
    return QASR_OK;
}

int qasr_plan_prefill(int rows, int kv_start, int nkvh, int32_t* rows_per_block, int32_t* nrb,
                      int32_t* tiles_per_split, int32_t* sp_base_out) {
    if (rows < 1 || rows > qasr::kMaxRowBlocks * qasr::kPrefillRows)
        return fail(QASR_EINVAL, "rows %d outside [1, %d]", rows, qasr::kMaxRowBlocks * qasr::kPrefillRows);
    if (kv_start < 0 || kv_start > kMaxPositions || nkvh < 1 || nkvh > 64)
        return fail(QASR_EINVAL, "kv_start %d / nkvh %d", kv_start, nkvh);
    if (!rows_per_block || !nrb || !tiles_per_split || !sp_base_out) return fail(QASR_EINVAL, "null pointer");
    const qasr::PrefillPlan P = choose_prefill_plan(rows, kv_start, nkvh, env_int("QASR_PREFILL_TPS", 0));
    *rows_per_block = P.rows_per_block;
    *nrb = P.nrb;
    *tiles_per_split = P.tps;
    for (int i = 0; i <= P.nrb; ++i) sp_base_out[i] = P.sp_base[i];
    return QASR_OK;
}

int qasr_prefill_layer(qasr_ctx* ctx, qasr_kv* kv, int layer, int slot, int kv_start, int s,
                       const void* qkv_dev, const void* q_gain_dev, const void* k_gain_dev,
                       void* q_work_dev, void* out_dev, void* stream) {
    qasr_segment seg{slot, kv_start, s};
    int rc = qasr_qk_norm_rope_append(ctx, kv, layer, &seg, 1, qkv_dev, q_gain_dev, k_gain_dev,
                                      q_work_dev, stream);
    if (rc) return rc;
    return qasr_prefill_attn(ctx, kv, layer, slot, kv_start, s, q_work_dev, out_dev, stream);
}

}  // extern "C"
