/*
 * qasr_attn.h -- C ABI of the MI355X (gfx950) Qwen3-ASR decoder self-attention
 * path: fused q/k-RMSNorm + MRoPE + fp16 KV append, GQA decode attention over
 * ragged per-slot contexts, and causal (chunked) prefill attention.
 *
 * The reference (eclipse005/qwen3-asr-wgpu, Rust + WGSL) has no plugin or FFI
 * around attention: its seam is the `TextBackend` enum (src/inference.rs:
 * 213-269) whose GPU arm runs the attention blocks inside WgpuTextDecoder.
 * Each entry point below names the reference code it replaces.  A Rust host
 * binds these with `extern "C"` declarations, the way src/mel.rs:544-566 binds
 * the vendored soxr C library.
 *
 * Conventions
 *  - Every function returns an int status (QASR_OK == 0); on failure
 *    qasr_last_error() returns a thread-local message.  Nothing throws across
 *    the ABI.
 *  - Tensor arguments named `*_dev` are device pointers (f16 stored as raw
 *    binary16 bits).  Arrays of slot ids, positions and lengths are HOST
 *    pointers: the host plans the launch from them, as the reference's host
 *    writes its per-step uniforms (decoder.rs:1674-1714, 3348-3379).
 *  - Work is stream-ordered and asynchronous on `stream` (a hipStream_t; NULL
 *    is the null stream).  A context and its KV pools are not thread-safe: one
 *    host thread drives a context, as the reference serialises decoder calls
 *    behind a Mutex (inference.rs:307-323).  Calls that share a KV pool must
 *    be ordered on one stream (they share its split-K workspace).
 *  - Head layout: head_dim must be 128 and num_attention_heads must be twice
 *    num_key_value_heads (both Qwen3-ASR sizes: 16 q heads, 8 kv heads).
 */
#ifndef QASR_ATTN_H
#define QASR_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QASR_ABI_VERSION 2

/* Status codes. */
#define QASR_OK 0
#define QASR_EINVAL 1   /* bad argument or unsupported shape */
#define QASR_ERANGE 2   /* position / length beyond capacity, max_seq or tables */
#define QASR_ENOMEM 3   /* device allocation failed */
#define QASR_EDEVICE 4  /* HIP runtime error */
#define QASR_ESTATE 5   /* call out of order (e.g. no RoPE tables yet) */

/* KV_INITIAL_CAP / KV_STEP (decoder.rs:716-725), DECODER_MAX_SEQ (inference.rs:19). */
#define QASR_KV_INITIAL_CAP 1024
#define QASR_KV_STEP 256
#define QASR_DECODER_MAX_SEQ 16384

/* Text decoder attention hyper-parameters (TextConfig, decoder.rs:164-174). */
typedef struct qasr_attn_cfg {
    int32_t num_attention_heads; /* 16 */
    int32_t num_key_value_heads; /* 8 */
    int32_t head_dim;            /* 128 */
    int32_t num_hidden_layers;   /* 28 */
    float rms_norm_eps;          /* 1e-6 */
    int32_t max_seq;             /* ceiling on positions (DECODER_MAX_SEQ); 1 .. 1 << 24 */
} qasr_attn_cfg;

typedef struct qasr_ctx qasr_ctx;
typedef struct qasr_kv qasr_kv;

/* A run of consecutive positions of one slot: rows pos0 .. pos0+rows-1.
 * A decode batch is one 1-row segment per slot; a prefill is one segment. */
typedef struct qasr_segment {
    int32_t slot;
    int32_t pos0;
    int32_t rows;
} qasr_segment;

/* Device layout of a KV pool, for callers that read or seed the cache.
 * Element (slot, layer, kv, head, pos, d), kv 0 = K and 1 = V, f16 at
 *   base + ((((slot*layers + layer)*2 + kv)*nkvh + head)*cap + pos)*head_dim + d
 * i.e. each (slot, layer) holds the reference's per-layer K and V buffers,
 * [nkvh][cap][head_dim] f16 (decoder.rs:1270-1271, index (kvh*cap+pos)*hd). */
typedef struct qasr_kv_info {
    void* base_dev;
    int32_t slots;
    int32_t layers;
    int32_t nkvh;
    int32_t cap;
    int32_t head_dim;
    int64_t slot_stride;  /* elements */
    int64_t layer_stride; /* elements */
    int64_t kv_stride;    /* elements, K block -> V block */
    int64_t head_stride;  /* elements (= cap * head_dim) */
    size_t bytes;
} qasr_kv_info;

int qasr_abi_version(void);
const char* qasr_last_error(void);

/* Context: binds a device and the shape.  Replaces WgpuTextDecoder::load's
 * attention-side setup (decoder.rs:977-1246). */
int qasr_ctx_create(const qasr_attn_cfg* cfg, int device, qasr_ctx** out);
void qasr_ctx_destroy(qasr_ctx* ctx);

/* MRoPE cos/sin tables for text positions 0..rows-1, rounded to f16
 * ([rows][head_dim] each).  Host-only.  Replaces compute_mrope_cos_sin +
 * text_positions + the f16 cast (mrope.rs:5-80, inference.rs:1038-1049). */
int qasr_mrope_text_tables(int rows, int head_dim, double rope_theta,
                           const int32_t* mrope_section, int nsec, int interleaved,
                           uint16_t* cos_f16, uint16_t* sin_f16);

/* Upload f16 tables ([rows][head_dim], host).  Replaces set_rope_tables
 * (decoder.rs:1664-1667; cpu_decoder.rs:215-221). */
int qasr_set_rope_tables(qasr_ctx* ctx, const uint16_t* cos_f16, const uint16_t* sin_f16,
                         int rows);

/* KV pool of `slots` sequences x all layers, capacity rounded up to KV_STEP.
 * Replaces the per-layer k_cache/v_cache buffers and fork_capped's per-slot
 * KV (decoder.rs:1270-1271, 1422-1423, 2453-2457). */
int qasr_kv_create(qasr_ctx* ctx, int slots, int cap, qasr_kv** out);
void qasr_kv_destroy(qasr_kv* kv);
int qasr_kv_get_info(const qasr_kv* kv, qasr_kv_info* out);

/* Grow-only capacity change, KV_STEP granular, clamped to max_seq; rows
 * 0..keep_rows-1 of every (slot, layer, head) are preserved.  Synchronous.
 * Replaces WgpuTextDecoder::ensure_capacity (decoder.rs:1604-1661). */
int qasr_kv_ensure_capacity(qasr_kv* kv, int need, int keep_rows, int* cap_out);

/* Stage (a): per row, RMSNorm each q and k head (gain q_gain / k_gain, f16
 * [head_dim]), rotate-half RoPE at the row's position, round to f16; roped Q
 * -> q_out_dev [rows][nqh*hd]; roped K and raw V -> the pool at (slot, layer,
 * pos).  qkv_dev holds the segments' rows back to back, fused [q | k | v]
 * ((nqh + 2*nkvh)*hd f16 per row).  Bit-identical to cpu_decoder.rs:274-290 +
 * 398-423.  Replaces qkv_extract / qkv_extract_slots (shaders.rs:1376-1635,
 * dispatched at decoder.rs:1813-1817, 3414-3421, 4871-4873). */
int qasr_qk_norm_rope_append(qasr_ctx* ctx, qasr_kv* kv, int layer,
                             const qasr_segment* segs, int nseg,
                             const void* qkv_dev, const void* q_gain_dev,
                             const void* k_gain_dev, void* q_out_dev, void* stream);

/* Stage (b): decode attention.  Batch entry b reads roped q_dev[b] ([nqh][hd])
 * against keys 0..cur_len[b]-1 of slot slots[b] (NULL: slot b) and writes
 * out_dev[b] ([nqh*hd] f16).  Split-K over the context with an in-kernel
 * merge.  Replaces encode_gqa / gqa_decode_single[_slots] /
 * gqa_decode_split_p1_pair / gqa_split_merge (decoder.rs:1959-2025, 3426-3451;
 * shaders.rs:1881-2905); semantics of cpu_decoder.rs:292-365 with rows = 1. */
int qasr_decode_attn(qasr_ctx* ctx, qasr_kv* kv, int layer, int batch, const int32_t* slots,
                     const int32_t* cur_len, const void* q_dev, void* out_dev, void* stream);

/* Stages (a)+(b) fused into one launch for one decode step of one layer:
 * batch entry b takes the raw qkv row qkv_dev[b] at position pos[b] of slot
 * slots[b], appends its roped K and raw V at pos[b], and attends keys
 * 0..pos[b].  Replaces the Extract + Gqa blocks of encode_into
 * (decoder.rs:1813-1829) and of BatchProjections::step (decoder.rs:3412-3451). */
int qasr_decode_step(qasr_ctx* ctx, qasr_kv* kv, int layer, int batch, const int32_t* slots,
                     const int32_t* pos, const void* qkv_dev, const void* q_gain_dev,
                     const void* k_gain_dev, void* out_dev, void* stream);

/* Stage (c): causal prefill attention of s rows at positions kv_start ..
 * kv_start+s-1 of one slot, against cache rows 0..kv_start+s-1 (rows written
 * by stage (a) beforehand).  q_dev [s][nqh*hd] roped, out_dev [s][nqh*hd].
 * kv_start > 0 is chunked prefill / KV-prefix reuse (stream.rs:366-376).
 * Replaces repeat_kv + prefill_gemm_causal + softmax_causal +
 * prefill_gemm_causal_av and the slab path (decoder.rs:4856-5098,
 * 3860-4005; shaders.rs:3058-4184). */
int qasr_prefill_attn(qasr_ctx* ctx, qasr_kv* kv, int layer, int slot, int kv_start, int s,
                      const void* q_dev, void* out_dev, void* stream);

/* Stage (c) exactly as qasr_prefill_attn, with no allocation of any kind
 * (no hipMalloc / hipFree, nothing a library allocates), for callers that
 * cannot allocate: code under HIP graph capture, tight serving loops,
 * harnesses that forbid it.  No counterpart in the reference.  The split-K
 * partials live in a static device array of the library (17.3 MB per GPU,
 * held until the process ends) instead of the KV pool's workspace, which
 * qasr_prefill_attn grows on demand.  Limits: s <= 64 * min(64, 256 / nkvh)
 * rows per call (2048 for 8 kv heads; longer prompts go in chunks with
 * kv_start > 0), nkvh <= 16; beyond them QASR_EINVAL.  Every call on one GPU
 * shares that array: calls that overlap on one GPU (different streams or
 * threads) race and must be serialised by the caller. */
int qasr_prefill_attn_noalloc(qasr_ctx* ctx, qasr_kv* kv, int layer, int slot, int kv_start,
                              int s, const void* q_dev, void* out_dev, void* stream);

/* Stage (c) for several segments in one call (the attention loop of
 * prefill_multi, decoder.rs:3642-3700, one dispatch per segment there):
 * segment i's roped q rows are rows row_i .. of q_dev (segments concatenated
 * in order), its output the same rows of out_dev, at positions
 * segs[i].pos0 .. of slot segs[i].slot, whose K/V are already appended.
 * Segments of short key ranges go out in one launch; the rest as in
 * qasr_prefill_attn.  Same checks as qasr_prefill_attn, before any launch. */
int qasr_prefill_attn_batch(qasr_ctx* ctx, qasr_kv* kv, int layer, const qasr_segment* segs,
                            int nseg, const void* q_dev, void* out_dev, void* stream);

/* Stages (a)+(c) for one layer of one slot's prefill: stage (a) on s raw qkv
 * rows (q_work_dev receives the roped Q, [s][nqh*hd]), then stage (c).
 * Replaces prefill_impl's attention block (decoder.rs:4856-5098). */
int qasr_prefill_layer(qasr_ctx* ctx, qasr_kv* kv, int layer, int slot, int kv_start, int s,
                       const void* qkv_dev, const void* q_gain_dev, const void* k_gain_dev,
                       void* q_work_dev, void* out_dev, void* stream);

/* ---- Whole text decoder around the attention path ------------------------
 * The layer sequence of src/cpu_decoder.rs:367-532 (CpuTextDecoder::forward,
 * final_norm_logits, argmax, prefill, step), i.e. what WgpuTextDecoder::step
 * and ::prefill run on the GPU (decoder.rs:1768-1925, 4489-5244): input
 * RMSNorm, fused q/k/v projection, stages (a)+(b) or (a)+(c) of this library,
 * o_proj + residual, post-attention RMSNorm, gate/up projection, SiLU(gate)*up,
 * down_proj + residual; final RMSNorm, logits against the tied embedding and
 * the greedy argmax.  Rounding follows the reference: f32 math, one f16
 * rounding per op output (a residual add rounds x + dot once), f32 logits,
 * the first maximal index on ties.  The projections run this library's own
 * MFMA kernels with f32 accumulation: the skinny decode-step kernels and, for
 * prefill, the tiled GEMM of gemm.hip (QASR_PREFILL_GEMM=blas: rocBLAS
 * instead); their summation order differs from the reference's, so logits
 * agree to rounding, not bitwise.  The order is fixed per shape (it never
 * depends on how many rows or slots a call carries), so a slot's or a
 * prompt's results are the same bits alone and in any batch.
 *
 * Weights are device pointers owned by the caller and must outlive the
 * decoder; f16 bits, row-major [out][in] as in the checkpoint.  A projection
 * whose *_scale pointer is set is int8 instead (the reference's resident-int8
 * checkpoints, weights.rs:296-427, decoder.rs:4364-4395): signed int8
 * [out][in] with one f32 scale per output row, each weight used as
 * f16(q * scale[row]) rounded to nearest even -- the value the reference's
 * W8 kernels form per weight.  Fused rows keep their parts' order for the
 * scales too. */
typedef struct qasr_layer_weights {
    const void* input_norm;   /* [hs] (input_layernorm) */
    const void* qkv_proj;     /* [(nqh + 2*nkvh)*hd][hs]: q_proj rows, then k_proj, then v_proj */
    const void* q_norm;       /* [hd] */
    const void* k_norm;       /* [hd] */
    const void* o_proj;       /* [hs][nqh*hd] */
    const void* post_norm;    /* [hs] (post_attention_layernorm) */
    const void* gate_up_proj; /* [2*inter][hs]: gate_proj rows, then up_proj */
    const void* down_proj;    /* [hs][inter] */
    const float* qkv_scale;     /* NULL, or [(nqh + 2*nkvh)*hd]: qkv_proj is int8 */
    const float* o_scale;       /* NULL, or [hs]: o_proj is int8 */
    const float* gate_up_scale; /* NULL, or [2*inter]: gate_up_proj is int8 */
    const float* down_scale;    /* NULL, or [hs]: down_proj is int8 */
} qasr_layer_weights;

typedef struct qasr_decoder_cfg {
    int32_t hidden_size;       /* 1024 (0.6B) or 2048 (1.7B) */
    int32_t intermediate_size; /* 3072 or 6144 */
    int32_t vocab_size;        /* 151936 */
    int32_t max_rows;          /* largest decode batch or prefill chunk one call runs (<= 16384) */
} qasr_decoder_cfg;

typedef struct qasr_decoder qasr_decoder;

/* embed_dev: [vocab][hs] (embed_tokens, also the tied lm_head);
 * final_norm_dev: [hs]; layers: num_hidden_layers entries (a host array, read
 * during the call).  Allocates the activation workspace for max_rows rows. */
int qasr_decoder_create(qasr_ctx* ctx, const qasr_decoder_cfg* cfg, const void* embed_dev,
                        const void* final_norm_dev, const qasr_layer_weights* layers,
                        qasr_decoder** out);
void qasr_decoder_destroy(qasr_decoder* dec);

/* One greedy step for `batch` slots (the reference's step(), and --batch N
 * through BatchProjections::step, decoder.rs:3348-3451): embeds
 * tokens_dev[b] (int32, device; ids outside [0, vocab) read row 0), runs every
 * layer at position pos[b] of slots[b] (host arrays; slots NULL = 0..batch-1)
 * and writes the argmax token of each entry to next_dev[b] (int32, device).
 * logits_dev, if not NULL, receives the f32 logits [batch][vocab]. */
int qasr_decoder_step(qasr_decoder* dec, qasr_kv* kv, int batch, const int32_t* slots,
                      const int32_t* pos, const int32_t* tokens_dev, int32_t* next_dev,
                      float* logits_dev, void* stream);

/* Prefill of s hidden rows ([s][hs] f16, device; the reference's
 * prefill(hidden_words, s, kv_start)) into `slot` at positions kv_start ..
 * kv_start+s-1 through every layer; next_dev[0] receives the argmax token of
 * the last row, logits_dev (optional) its f32 logits [vocab].  s <= max_rows;
 * longer prompts are prefilled in chunks (kv_start > 0). */
int qasr_decoder_prefill(qasr_decoder* dec, qasr_kv* kv, int slot, int kv_start, int s,
                         const void* hidden_dev, int32_t* next_dev, float* logits_dev,
                         void* stream);

/* Prefill of several segments at once (prefill_batch / prefill_multi,
 * decoder.rs:3599-3700): segment i writes segs[i].rows rows into slot
 * segs[i].slot at positions segs[i].pos0 ..; the hidden rows of all segments
 * are concatenated in segment order ([sum rows][hs] f16, device).  Every
 * projection runs once over all rows (row-independent), attention per
 * segment; next_dev[i] receives the argmax token after segment i's last row,
 * logits_dev (optional) its f32 logits [nseg][vocab].  Slots must be
 * distinct, every segment at least one row, the rows together <= max_rows. */
int qasr_decoder_prefill_batch(qasr_decoder* dec, qasr_kv* kv, const qasr_segment* segs,
                               int nseg, const void* hidden_dev, int32_t* next_dev,
                               float* logits_dev, void* stream);

/* out[r][c] = f16(f32(q[r][c]) * scale[r]) with RNE (dequant_i8,
 * weights.rs:366-385): the f16 copy of a resident-int8 checkpoint weight,
 * the same values the decoder's int8 projections compute with.  q (int8
 * [rows][cols]), scale (f32 [rows]) and out (f16 [rows][cols]) are device
 * pointers on ctx's device; cols a multiple of 8, q 8-byte and out 16-byte
 * aligned. */
int qasr_dequant_i8(qasr_ctx* ctx, const void* q_dev, const float* scale_dev, int64_t rows,
                    int32_t cols, void* out_dev, void* stream);

/* c[m][n] = f16(sum_k a[m][k] * b[n][k] (+ c[m][n] when accumulate)), f32
 * accumulation and one rounding: the prefill projections' GEMM (the
 * reference's tiled prefill GEMMs, shaders.rs:3033-3105 and 3105-3727,
 * dispatched by decoder.rs:3580-4162; rounding as batch_dot_acc,
 * cpu_decoder.rs:45-62).  a [m][k] (activation rows), b [n][k] (weight rows,
 * checkpoint layout) and c [m][n] are f16 device pointers on ctx's device,
 * 16-byte aligned; k a multiple of 64, n a multiple of 256, a and b each
 * under 2 GB.  Every output sums over k in one fixed order whatever m is,
 * so a row's result does not depend on the other rows of the call (the
 * block tile, chosen per shape, never changes a bit). */
int qasr_gemm_f16(qasr_ctx* ctx, const void* a_dev, const void* b_dev, void* c_dev, int32_t m,
                  int32_t n, int32_t k, int accumulate, void* stream);

/* Diagnostic: the attention kernels' softmax weight for scores s_dev[i]
 * against row maxima m_dev[i] (f32, device, n each; m >= s), in both forms
 * the kernels use: out_scaled_dev[i] = 2^(f32(s*sl2) - f32(m*sl2)) (decode)
 * and out_raw_dev[i] = 2^(fma(s, sl2, -f32(m*sl2))) (prefill), where sl2 =
 * the context's softmax scale times log2(e).  The reference forms
 * expf(f32(s*scale) - f32(m*scale)) (cpu_decoder.rs:292-365); this entry
 * exists so tests can measure the difference.  No counterpart in the
 * reference. */
int qasr_softmax_weights(qasr_ctx* ctx, const float* s_dev, const float* m_dev, int64_t n,
                         float* out_scaled_dev, float* out_raw_dev, void* stream);

/* Calibration: a bare streaming read of `bytes` bytes at src_dev (device)
 * by `wgs` workgroups of `waves` waves, each reading one contiguous share
 * with the decode kernel's load form (non-temporal dwordx4 buffer loads);
 * sink_dev receives one word per wave (wgs * waves uint32).  bytes must be a
 * multiple of 16 * wgs.  Measures what the memory system delivers to one
 * launch of a given size, against which the decode kernel's bandwidth is
 * read.  No counterpart in the reference. */
int qasr_stream_read(qasr_ctx* ctx, const void* src_dev, int64_t bytes, int wgs, int waves,
                     uint32_t* sink_dev, void* stream);

/* Calibration: `wgs` workgroups of `waves` waves (8 for mode 2) run
 * mfma_iters iterations of four independent v_mfma_f32_32x32x16_f16 chains
 * and/or valu_iters iterations of a softmax-shaped VALU block (16 values: row
 * max, FMA + v_exp_f32 each, packed f16 conversion, v_dot2 sum).  mode % 4
 * = 0: MFMA only; 1: VALU only; 2: waves 0-3 MFMA and waves 4-7 VALU (one of
 * each per SIMD); 3: both interleaved in every wave.  mode / 4 picks the VALU
 * block: 0 the whole mix; 1 exponentials only; 2 FMAs only; 3 v_dot2 only;
 * 4 packed f16 conversions only; 5 v_max3 only; 6 the mix with f32 adds for
 * the row sum; 7 the mix with single f16 conversions.  sink_dev receives one float
 * per wave (wgs * waves), clk_dev four uint64: s_memtime and s_memrealtime
 * (100 MHz) of wave 0 of workgroup 0 at its start and end.  Measures what the
 * prefill kernel's MFMA roofline and its softmax/MFMA overlap are read
 * against.  No counterpart in the reference. */
int qasr_mfma_probe(qasr_ctx* ctx, int mode, int wgs, int waves, int mfma_iters, int valu_iters,
                    float* sink_dev, unsigned long long* clk_dev, void* stream);

/* Launch planning on the host, for tests (no device, no context): the
 * split plans the decode and prefill entry points launch with.  No
 * counterpart in the reference (its chunk choice is decoder.rs:899-916,
 * 1932-1957; its prefill dispatch has no key split).
 *
 * Decode (qasr_decode_attn / qasr_decode_step): `batch` (1..64) entries
 * attending lens[b] >= 1 keys, `nkvh` kv heads, a device of `cus` compute
 * units; the QASR_DECODE_WGS / _GRANULE / _MAX_GRANULES environment knobs
 * apply.  gran_out[b]: keys per granule of entry b (a multiple of 256 and a
 * function of lens[b] alone: the entry's output bits do not depend on its
 * batch mates); run_out[b]: granules per workgroup; wg_base_out[0..batch]:
 * entry b's workgroups are wg_base_out[b] .. wg_base_out[b+1]-1
 * (nkvh * ceil(ceil(lens[b] / gran_out[b]) / run_out[b]) of them).
 * lens[b] in [1, 1 << 24]. */
int qasr_plan_decode(int batch, const int32_t* lens, int nkvh, int cus, int32_t* gran_out,
                     int32_t* run_out, int32_t* wg_base_out);

/* Prefill (qasr_prefill_attn, one launch of 1..4096 rows at kv_start):
 * *rows_per_block (64; 32 or 16 for unsplit short key ranges), *nrb row
 * blocks, *tiles_per_split 128-key tiles per split (QASR_PREFILL_TPS
 * applies), sp_base_out[0..nrb]: row block rb's items are sp_base_out[rb] ..
 * sp_base_out[rb+1]-1 within each kv head (sp_base_out[nrb] items per kv
 * head; at most 65 entries written).  kv_start in [0, 1 << 24]. */
int qasr_plan_prefill(int rows, int kv_start, int nkvh, int32_t* rows_per_block, int32_t* nrb,
                      int32_t* tiles_per_split, int32_t* sp_base_out);

#ifdef __cplusplus
}
#endif
#endif /* QASR_ATTN_H */
