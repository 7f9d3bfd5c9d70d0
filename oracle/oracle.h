/*
 * oracle.h -- CPU restatement of Qwen3-ASR's decoder self-attention path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or the timed CPU baseline).  The shipped HIP library never links it.
 *
 * Every function restates one piece of the reference (eclipse005/qwen3-asr-wgpu,
 * Rust) in C++, in the reference's own operation order, compiled with
 * -ffp-contract=off and without fast-math so each float operation rounds the
 * way the Rust source does (Rust never contracts a*b+c into an FMA).
 *
 * Reference files (paths under the reference checkout):
 *   src/cpu_decoder.rs  : norm_rope_head 274-290, attention 292-365,
 *                         KV write 398-423, set_rope_tables 215-221,
 *                         ensure_capacity 227-249
 *   src/mrope.rs        : build_dim_map 5-41, compute_mrope_cos_sin 46-74,
 *                         text_positions 77-80
 *   src/inference.rs    : f16 table rounding 1041-1051
 *   src/decoder.rs      : KV_INITIAL_CAP / KV_STEP 716-725, scale 204-206
 *   half 2.7.1          : f16::from_f32 / to_f32 (IEEE binary16, RNE, subnormals)
 */
#ifndef QASR_ORACLE_H
#define QASR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- IEEE binary16 conversions (half 2.7.1 semantics) ------------------ */
uint16_t qo_f16_from_f32(float f);
float qo_f32_from_f16(uint16_t h);
void qo_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n);
void qo_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n);

/* ---- MRoPE tables (mrope.rs) -------------------------------------------- */
/* build_dim_map: out[half] = axis index per frequency (mrope.rs:5-41). */
int qo_build_dim_map(const int32_t* section, int nsec, int half, int interleaved, int32_t* out);
/* compute_mrope_cos_sin over 3 position axes pos3[3][n] -> f32 [n][head_dim]
 * (mrope.rs:46-74). */
int qo_mrope_cos_sin(const int64_t* pos3, int n, int head_dim, double theta,
                     const int32_t* section, int nsec, int interleaved,
                     float* cos_out, float* sin_out);
/* The text-position tables the decoder consumes, rounded to f16
 * (mrope.rs:77-80 + inference.rs:1041-1051). */
int qo_text_rope_tables_f16(int rows, int head_dim, double theta,
                            const int32_t* section, int nsec, int interleaved,
                            uint16_t* cos_f16, uint16_t* sin_f16);

/* ---- per-head q/k RMSNorm + rotate-half RoPE (cpu_decoder.rs:274-290) --- */
void qo_norm_rope_head(const uint16_t* raw, const float* gain, const float* cos_row,
                       const float* sin_row, int hd, float eps, uint16_t* out);

/* ---- one decoder layer's attention path for one sequence ----------------
 * Restates cpu_decoder.rs forward() lines 398-427 for a run of `rows`
 * consecutive positions q0..q0+rows-1 of one sequence:
 *   q heads  -> norm_rope_head -> q_out (f16)            (401-409)
 *   k heads  -> norm_rope_head -> k_cache[h][pos] (f32)  (410-417)
 *   v heads  -> v_cache[h][pos] (f32)                    (418-421)
 *   attention(q, q0) -> attn_out (f16)                   (292-365, 427)
 * qkv rows are the fused [q | k | v] layout, (nqh + 2*nkvh)*hd f16 per row.
 * k_cache / v_cache are this layer's [nkvh][cap][hd] f32 blocks.
 * cos/sin are the f32 values of the f16 tables, [tab_rows][hd].
 * nthreads <= 0 means one worker per logical CPU.  Returns 0 or -1. */
typedef struct qo_shape {
    int32_t nqh;
    int32_t nkvh;
    int32_t hd;
    int32_t max_seq;
    float eps;
} qo_shape;

int qo_layer_attn(const qo_shape* sh, int cap, const uint16_t* qkv, int rows, int q0,
                  const uint16_t* q_gain, const uint16_t* k_gain,
                  const float* cos_tab, const float* sin_tab, int tab_rows,
                  float* k_cache, float* v_cache, uint16_t* q_out, uint16_t* attn_out,
                  int nthreads);

/* Stage (a) only (cpu_decoder.rs:398-423): q_out, k_cache, v_cache. */
int qo_qk_norm_rope_append(const qo_shape* sh, int cap, const uint16_t* qkv, int rows, int q0,
                           const uint16_t* q_gain, const uint16_t* k_gain,
                           const float* cos_tab, const float* sin_tab, int tab_rows,
                           float* k_cache, float* v_cache, uint16_t* q_out);

/* Attention only (cpu_decoder.rs:292-365): q is roped f16 [rows][nqh*hd]. */
int qo_attention(const qo_shape* sh, int cap, const uint16_t* q, int rows, int q0,
                 const float* k_cache, const float* v_cache, uint16_t* attn_out, int nthreads);

/* ensure_capacity's target rule (cpu_decoder.rs:227-229, decoder.rs:1610). */
int qo_kv_target_cap(int need, int cap, int max_seq);

/* ---- seeded synthetic inputs (this build's generator, not the reference's) --
 * SplitMix64 stream; N(mean, std) by Box-Muller in f64 -> f32 -> f16 RNE. */
uint64_t qo_splitmix64(uint64_t* state);
void qo_fill_normal_f16(uint64_t* state, int64_t n, double mean, double std, uint16_t* out);
int32_t qo_uniform_int(uint64_t* state, int32_t lo, int32_t hi); /* inclusive */

int qo_hardware_threads(void);

/* Softmax weight of the reference attention (cpu_decoder.rs:292-365) for a
 * raw dot product s against the row's largest dot m: out[i] =
 * expf(f32(s*scale) - f32(m*scale)), glibc expf, each operation rounded as
 * the Rust source rounds it. */
void qo_softmax_weights(const float* s, const float* m, int64_t n, float scale, float* out);

/* ---- the whole text decoder for one sequence (cpu_decoder.rs) -----------
 * CpuTextDecoder restated for the end-to-end greedy check: rms_norm_row
 * 261-272, forward 367-456 (q/k/v/o/gate/up/down with dot_transposed's
 * 4-way partial sums 64-100, f16 after every projection and residual add,
 * SiLU), final_norm_logits 458-472 (tied embedding), argmax 474-482 (first
 * maximum), prefill 487-516, step 518-532.  Rows >= 2 of a prefill use the
 * one-row summation order (the reference calls the gemm crate there).
 * layer_ptrs: 11 f16 tensors per layer, checkpoint layout [out][in]:
 *   input_layernorm[hs], post_attention_layernorm[hs], q_norm[hd], k_norm[hd],
 *   q_proj[nqh*hd][hs], k_proj[nkvh*hd][hs], v_proj[nkvh*hd][hs],
 *   o_proj[hs][nqh*hd], gate_proj[inter][hs], up_proj[inter][hs],
 *   down_proj[hs][inter].
 * The decoder reads the weight arrays in place: the caller keeps them alive
 * until qo_dec_destroy.  The KV caches hold `cap` positions per layer (no
 * growth). */
typedef struct qo_dec_cfg {
    int32_t hs;
    int32_t nqh;
    int32_t nkvh;
    int32_t hd;
    int32_t inter;
    int32_t layers;
    int32_t vocab;
    int32_t max_seq;
    float eps;
} qo_dec_cfg;

void* qo_dec_create(const qo_dec_cfg* cfg, const uint16_t* embed, const uint16_t* final_norm,
                    const uint16_t* const* layer_ptrs, int cap);
void qo_dec_destroy(void* d);
int qo_dec_set_rope(void* d, const uint16_t* cos_f16, const uint16_t* sin_f16, int rows);
/* Returns the argmax token of the last row (or -1); logits may be NULL. */
int qo_dec_prefill(void* d, const uint16_t* hidden, int s, int kv_start, float* logits);
/* Embeds the previous argmax token and runs one position. */
int qo_dec_step(void* d, float* logits);
int qo_dec_pos(void* d);

#ifdef __cplusplus
}
#endif
#endif
