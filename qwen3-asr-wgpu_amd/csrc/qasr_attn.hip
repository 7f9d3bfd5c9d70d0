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

// Decode workspace: one partial per workgroup of a launch (the planner keeps a
// launch under kDecodeMaxItems workgroups) and one ticket per (entry, kv head).
int alloc_decode_ws(qasr_kv* kv) {
    const int nkvh = kv->ctx->cfg.num_key_value_heads;
    const int64_t items = qasr::kDecodeMaxItems;
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
    const size_t cbytes = (size_t)nkvh * qasr::kMaxRowBlocks * sizeof(uint32_t);
    HIP_TRY(hipMalloc(&kv->pws_ctr, cbytes), "prefill counters");
    HIP_TRY(hipMemset(kv->pws_ctr, 0, cbytes), "prefill counters");
    kv->pws_items = items;
    return QASR_OK;
}

// Decode launch plan: a fixed number of workgroups (QASR_DECODE_WGS, default
// one per CU), each streaming one chunk of one entry's keys for one kv head.
// One CU streams at most ~45-70 GB/s (a bare stream measures the same), so
// a CU cannot speed up when others finish: the launch ends at full HBM
// rate only while enough CUs are still streaming.  So when the batch leaves
// room to split (entries x kv heads below the budget), every entry is cut
// into chunks of one common size C -- the smallest multiple of 32 keys that
// fits the budget (and at least QASR_DECODE_MIN_CHUNK keys, at most
// QASR_DECODE_MAX_SPLIT chunks per entry) -- plus a shorter last chunk, and
// entries shorter than C stay whole.  Most workgroups then carry C keys and
// stream until the end (config 3: 20.1 against 21.0 us for equal chunks
// within each entry, the plan before).  Batches at or past the budget split
// their longest entries while a chunk exceeds 1.5x the average keys per
// workgroup; the extra workgroups run as the first ones finish.
int chunk_of(int L, int n) {
    const int c = (L + n - 1) / n;
    return (c + qasr::kDecodeTileKeys - 1) / qasr::kDecodeTileKeys * qasr::kDecodeTileKeys;
}

void plan_decode_chunks(qasr::DecodePlan& P, int nkvh, int cus) {
    const int target = std::max(1, std::min(env_int("QASR_DECODE_WGS", cus), 4096));
    const int min_chunk = std::max(32, env_int("QASR_DECODE_MIN_CHUNK", qasr::kDecodeMinChunk));
    const int max_split = std::max(1, std::min(env_int("QASR_DECODE_MAX_SPLIT", qasr::kDecodeMaxSplit),
                                               qasr::kDecodeMaxChunksPerEntry));
    int n[qasr::kMaxBatch];  // chunks per entry (greedy plan)
    int wgs = 0;
    for (int i = 0; i < P.batch; ++i) {
        n[i] = 1;
        wgs += nkvh;
    }
    int common = 0;  // C of the common-size plan, 0 for the greedy plan
    if (wgs < target) {
        int c = chunk_of(min_chunk, 1);
        for (int i = 0; i < P.batch; ++i) c = std::max(c, chunk_of(P.len[i], max_split));
        auto items = [&](int cc) {
            int64_t t = 0;
            for (int i = 0; i < P.batch; ++i) t += (int64_t)nkvh * ((P.len[i] + cc - 1) / cc);
            return t;
        };
        while (items(c) > target) c += qasr::kDecodeTileKeys;
        common = c;
    } else {
        int64_t keys = 0;
        for (int i = 0; i < P.batch; ++i) keys += (int64_t)nkvh * P.len[i];
        while (wgs + nkvh <= qasr::kDecodeMaxItems / 2) {
            int best = -1, best_chunk = 0;
            for (int i = 0; i < P.batch; ++i) {
                const int c = chunk_of(P.len[i], n[i]);
                if (n[i] < max_split && chunk_of(P.len[i], n[i] + 1) >= min_chunk &&
                    c > best_chunk) {
                    best = i;
                    best_chunk = c;
                }
            }
            if (best < 0 || 2 * (int64_t)best_chunk * wgs <= 3 * keys) break;
            ++n[best];
            wgs += nkvh;
        }
    }
    P.wg_base[0] = 0;
    for (int i = 0; i < P.batch; ++i) {
        const int L = P.len[i];
        const int chunk = common ? std::min(common, chunk_of(L, 1)) : chunk_of(L, n[i]);
        P.chunk[i] = chunk;
        P.wg_base[i + 1] = P.wg_base[i] + nkvh * ((L + chunk - 1) / chunk);
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
        plan_decode_chunks(P, nkvh, ctx->cus);
        const f16* qp = (const f16*)qin + b0 * in_row;
        f16* op = (f16*)out + b0 * out_row;
        const int waves = env_int("QASR_DECODE_WAVES", qasr::kDecodeWaves);
        hipError_t e = qasr::launch_decode_attn(fused, waves, g, layer, P, P.wg_base[nb], qp,
                                                (const f16*)q_gain, (const f16*)k_gain, ctx->cos,
                                                ctx->sin, op, ws, (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "decode attention launch");
    }
    return QASR_OK;
}

// ---- prefill: planning shared by the allocating and the no-allocation entry

// Split workspace of qasr_prefill_attn_noalloc, for callers that cannot
// allocate (HIP graph capture, serving loops, harnesses that forbid it): a
// file-scope device array, one copy per GPU, alive until the process ends.
// Partials of at most kScratchItems work items (17.3 MB) plus the arrival
// counters.  Host code reaches it only through the address resolved per
// device by hipGetSymbolAddress (scratch_ptr); the array's name is a host
// stand-in, not a device address.
constexpr int64_t kScratchItems = 256;
constexpr int kScratchMaxKvHeads = 16;  // nkvh <= 16 (qasr_ctx_create's head limit)
constexpr int64_t kScratchO = kScratchItems * qasr::kPrefillItemFloats;
constexpr int64_t kScratchMl = kScratchItems * qasr::kPrefillItemMl;
constexpr int64_t kScratchCounters = (int64_t)kScratchMaxKvHeads * qasr::kMaxRowBlocks;
static __device__ __align__(256) float scratch[kScratchO + kScratchMl + kScratchCounters];

constexpr int kMaxDevices = 64;
constexpr int kPrefillNoSplitTiles = 4;  // key ranges of up to 512 keys run unsplit
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

// Longest prefill one qasr_prefill_attn_noalloc call takes: every row block
// of the launch must have at least one work item in the scratch array.
int noalloc_max_rows(int nkvh) {
    return qasr::kPrefillRows * (int)std::min<int64_t>(qasr::kMaxRowBlocks, kScratchItems / nkvh);
}

// The plan of one prefill launch of `rows` (<= kMaxRowBlocks * kPrefillRows)
// rows at kv_start `ks`.  Tiles per split: about one workgroup per CU (256),
// without splitting row blocks whose key range is short.  A split's merge
// (publish, ticket, read back) is about three memory round trips, as long as
// several latency-bound tiles: key ranges of up to kPrefillNoSplitTiles tiles
// are never split.  Unsplit short ranges also take 32-row blocks: twice the
// workgroups, half the work on the longest one.  A forced split count
// (tps_forced > 0, QASR_PREFILL_TPS) keeps 64-row blocks.
qasr::PrefillPlan choose_prefill_plan(int rows, int ks, int nkvh, int tps_forced) {
    const int nrb = (rows + qasr::kPrefillRows - 1) / qasr::kPrefillRows;
    const int max_tiles = (ks + rows + qasr::kPrefillTileKeys - 1) / qasr::kPrefillTileKeys;
    int tps = tps_forced;
    int rb_rows = qasr::kPrefillRows;
    if (tps <= 0) {
        const int64_t tiles_all = (int64_t)nrb * max_tiles;
        const int64_t want = std::max<int64_t>(1, 256 / nkvh);
        if (max_tiles <= kPrefillNoSplitTiles) {
            tps = max_tiles;
            rb_rows = qasr::kPrefillRows / 2;
        } else {
            tps = (int)std::max<int64_t>(2, (tiles_all + want - 1) / want);
        }
    }
    return qasr::plan_prefill(rows, ks, nkvh, tps, rb_rows);
}

int run_prefill(qasr_ctx* ctx, qasr_kv* kv, int layer, int slot, int kv_start, int s,
                const void* q_dev, void* out_dev, void* stream, bool noalloc) {
    int rc = check_common(ctx, kv, layer);
    if (rc) return rc;
    if (slot < 0 || slot >= kv->slots)
        return fail(QASR_EINVAL, "slot %d outside [0, %d)", slot, kv->slots);
    if (kv_start < 0 || s < 0) return fail(QASR_EINVAL, "negative kv_start / s");
    if (s == 0) return QASR_OK;
    if (!q_dev || !out_dev) return fail(QASR_EINVAL, "null device pointer");
    const int64_t end = (int64_t)kv_start + s;
    if (end > ctx->cfg.max_seq)
        return fail(QASR_ERANGE, "prefill needs %lld positions, max_seq is %d", (long long)end,
                    ctx->cfg.max_seq);
    if (end > kv->cap)
        return fail(QASR_ERANGE, "prefill needs %lld positions, KV capacity is %d",
                    (long long)end, kv->cap);
    const qasr_attn_cfg& c = ctx->cfg;
    const int nqh = c.num_attention_heads, nkvh = c.num_key_value_heads;
    if (noalloc) {
        if (nkvh > kScratchMaxKvHeads)
            return fail(QASR_EINVAL, "%d kv heads: the no-allocation prefill takes at most %d",
                        nkvh, kScratchMaxKvHeads);
        if (s > noalloc_max_rows(nkvh))
            return fail(QASR_EINVAL, "%d rows: the no-allocation prefill takes at most %d rows per "
                        "call (prefill longer prompts in chunks, kv_start > 0)", s,
                        noalloc_max_rows(nkvh));
        if (!ctx->scratch) return fail(QASR_ESTATE, "context has no prefill scratch address");
    }
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    const qasr::CacheGeom g = geom(kv);
    const int64_t ld = (int64_t)nqh * qasr::kHeadDim;
    const int rows_per_launch = qasr::kMaxRowBlocks * qasr::kPrefillRows;
    const int tps_forced = env_int("QASR_PREFILL_TPS", 0);
    qasr::PrefillWs fixed{};
    if (noalloc) {
        fixed.o = ctx->scratch;
        fixed.ml = ctx->scratch + kScratchO;
        fixed.counters = reinterpret_cast<uint32_t*>(ctx->scratch + kScratchO + kScratchMl);
        fixed.items = kScratchItems;
        // The array keeps the last call's contents: the arrival counters
        // start this call at zero.
        const int n = nkvh * qasr::kMaxRowBlocks;
        hipLaunchKernelGGL(zero_u32_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                           fixed.counters, n);
        HIP_TRY(hipGetLastError(), "scratch counter clear");
    }
    for (int r0 = 0; r0 < s; r0 += rows_per_launch) {
        const int rows = std::min(rows_per_launch, s - r0);
        const int ks = kv_start + r0;
        const int max_tiles = (ks + rows + qasr::kPrefillTileKeys - 1) / qasr::kPrefillTileKeys;
        qasr::PrefillPlan P = choose_prefill_plan(rows, ks, nkvh, tps_forced);
        int tps = P.tps;
        const int rb_rows = P.rows_per_block;
        if (noalloc) {
            // Coarser splits until the partials fit the scratch array; at
            // tps = max_tiles every row block is one item (s is bounded so
            // that this fits).
            while ((int64_t)P.items_per_kvh * nkvh > kScratchItems && tps < max_tiles) {
                tps = std::min(max_tiles, tps * 2);
                P = qasr::plan_prefill(rows, ks, nkvh, tps, rb_rows);
            }
            if ((int64_t)P.items_per_kvh * nkvh > kScratchItems)
                return fail(QASR_EINVAL, "prefill plan of %lld items exceeds the scratch's %lld",
                            (long long)P.items_per_kvh * nkvh, (long long)kScratchItems);
        } else {
            rc = ensure_prefill_ws(kv, (int64_t)P.items_per_kvh * nkvh);
            if (rc) return rc;
        }
        qasr::PrefillArgs a;
        a.q = (const f16*)q_dev + r0 * ld;
        a.out = (f16*)out_dev + r0 * ld;
        a.k = g.base + slot * g.slot_stride + layer * g.layer_stride;
        a.v = a.k + g.kv_stride;
        a.head_stride = g.head_stride;
        a.nqh = nqh;
        a.nkvh = nkvh;
        a.s = rows;
        a.kv_start = ks;
        a.scale_log2 = ctx->scale_log2;
        const qasr::PrefillWs ws =
            noalloc ? fixed : qasr::PrefillWs{kv->pws_o, kv->pws_ml, kv->pws_ctr, kv->pws_items};
        hipError_t e = qasr::launch_prefill_attn(a, P, ws, (hipStream_t)stream);
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
    return run_prefill(ctx, kv, layer, slot, kv_start, s, q_dev, out_dev, stream, false);
}

int qasr_prefill_attn_noalloc(qasr_ctx* ctx, qasr_kv* kv, int layer, int slot, int kv_start,
                              int s, const void* q_dev, void* out_dev, void* stream) {
    return run_prefill(ctx, kv, layer, slot, kv_start, s, q_dev, out_dev, stream, true);
}

// Longest key range (kv_start + rows) of a segment that a one-launch batched
// prefill takes: each row block's keys are then one workgroup's work.
constexpr int kPrefillOneLaunchKeys = 2048;

int qasr_prefill_attn_batch(qasr_ctx* ctx, qasr_kv* kv, int layer, const qasr_segment* segs,
                            int nseg, const void* q_dev, void* out_dev, void* stream) {
    int rc = check_common(ctx, kv, layer);
    if (rc) return rc;
    if (nseg < 0 || (nseg > 0 && !segs)) return fail(QASR_EINVAL, "bad segment list");
    if (nseg == 0) return QASR_OK;
    if (!q_dev || !out_dev) return fail(QASR_EINVAL, "null device pointer");
    // Every segment checked before any launch.  One launch takes them all
    // when each key range is short enough to be one workgroup's per row
    // block (no split); otherwise one launch per segment, which splits long
    // key ranges across workgroups.
    bool one_launch = nseg > 1 && nseg <= qasr::kMaxPrefillSegs;
    for (int i = 0; i < nseg; ++i) {
        const qasr_segment& g = segs[i];
        if (g.slot < 0 || g.slot >= kv->slots)
            return fail(QASR_EINVAL, "segment %d: slot %d outside [0, %d)", i, g.slot, kv->slots);
        if (g.pos0 < 0 || g.rows < 0) return fail(QASR_EINVAL, "segment %d: negative kv_start/rows", i);
        const int64_t end = (int64_t)g.pos0 + g.rows;
        if (end > ctx->cfg.max_seq)
            return fail(QASR_ERANGE, "segment %d: prefill needs %lld positions, max_seq is %d", i,
                        (long long)end, ctx->cfg.max_seq);
        if (end > kv->cap)
            return fail(QASR_ERANGE, "segment %d: prefill needs %lld positions, KV capacity is %d",
                        i, (long long)end, kv->cap);
        if (end > kPrefillOneLaunchKeys || g.rows > qasr::kMaxRowBlocks * qasr::kPrefillRows)
            one_launch = false;
    }
    const int64_t ld = (int64_t)ctx->cfg.num_attention_heads * qasr::kHeadDim;
    if (!one_launch) {
        int64_t r0 = 0;
        for (int i = 0; i < nseg; ++i) {
            rc = qasr_prefill_attn(ctx, kv, layer, segs[i].slot, segs[i].pos0, segs[i].rows,
                                   (const f16*)q_dev + r0 * ld, (f16*)out_dev + r0 * ld, stream);
            if (rc) return rc;
            r0 += segs[i].rows;
        }
        return QASR_OK;
    }
    DeviceScope ds(ctx->device);
    if (ds.err != hipSuccess) return hip_fail(ds.err, "hipSetDevice");
    const qasr_attn_cfg& c = ctx->cfg;
    const qasr::CacheGeom g = geom(kv);
    qasr::PrefillSegs S{};
    S.n = nseg;
    S.item_base[0] = 0;
    int32_t r0 = 0;
    for (int i = 0; i < nseg; ++i) {
        const int nrb = (segs[i].rows + qasr::kPrefillRows - 1) / qasr::kPrefillRows;
        S.item_base[i + 1] = S.item_base[i] + c.num_key_value_heads * nrb;
        S.kv_start[i] = segs[i].pos0;
        S.rows[i] = segs[i].rows;
        S.row_base[i] = r0;
        S.kv_off[i] = (int64_t)segs[i].slot * g.slot_stride + (int64_t)layer * g.layer_stride;
        r0 += segs[i].rows;
    }
    qasr::PrefillArgs a;
    a.q = (const f16*)q_dev;
    a.out = (f16*)out_dev;
    a.k = g.base;
    a.v = g.base + g.kv_stride;
    a.head_stride = g.head_stride;
    a.nqh = c.num_attention_heads;
    a.nkvh = c.num_key_value_heads;
    a.s = 0;
    a.kv_start = 0;
    a.scale_log2 = ctx->scale_log2;
    const hipError_t e = qasr::launch_prefill_attn_segs(a, S, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "prefill attention launch");
    return QASR_OK;
}

int qasr_plan_decode(int batch, const int32_t* lens, int nkvh, int cus, int32_t* chunk_out,
                     int32_t* wg_base_out) {
    if (batch < 1 || batch > qasr::kMaxBatch)
        return fail(QASR_EINVAL, "batch %d outside [1, %d]", batch, qasr::kMaxBatch);
    if (nkvh < 1 || nkvh > 64 || cus < 1) return fail(QASR_EINVAL, "nkvh %d / cus %d", nkvh, cus);
    if (!lens || !chunk_out || !wg_base_out) return fail(QASR_EINVAL, "null pointer");
    qasr::DecodePlan P{};
    P.batch = batch;
    for (int b = 0; b < batch; ++b) {
        if (lens[b] < 1 || lens[b] > kMaxPositions)
            return fail(QASR_EINVAL, "entry %d attends %d keys (at most %d)", b, lens[b], kMaxPositions);
        P.len[b] = lens[b];
    }
    plan_decode_chunks(P, nkvh, cus);
    for (int b = 0; b < batch; ++b) chunk_out[b] = P.chunk[b];
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
