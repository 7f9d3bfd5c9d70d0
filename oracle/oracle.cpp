// oracle.cpp -- CPU restatement of Qwen3-ASR's decoder self-attention path.
//
// TEST INFRASTRUCTURE, NOT PRODUCT CODE: the checker that tests/, smoke() and
// bench.py's cpu_baseline leg use.  The shipped HIP library never links it.
//
// Build: g++ -O3 -mf16c -ffp-contract=off -fno-fast-math (oracle/Makefile).  Without
// contraction every a*b+c below rounds twice, as in the Rust source it follows.
// std::exp(float) / std::sqrt(float) are glibc expf / IEEE sqrtf, the functions
// Rust's f32::exp / f32::sqrt call on Linux.

#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <functional>
#include <immintrin.h>
#include <mutex>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------
// A persistent worker pool, standing in for rayon's global pool (one worker per
// logical CPU by default).  parallel_for hands out task indices from an atomic
// counter; each task runs sequentially inside one worker, so results do not
// depend on the thread count (cpu_decoder.rs:301-364 is per-task sequential).
// ---------------------------------------------------------------------------
class Pool {
  public:
    explicit Pool(int n) : n_(n) {
        for (int i = 0; i < n_ - 1; ++i) workers_.emplace_back([this] { loop(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
            ++gen_;
        }
        cv_.notify_all();
        for (auto& t : workers_) t.join();
    }
    int size() const { return n_; }
    void run(int64_t ntasks, const std::function<void(int64_t)>& fn) {
        if (ntasks <= 0) return;
        if (n_ == 1 || ntasks == 1) {
            for (int64_t i = 0; i < ntasks; ++i) fn(i);
            return;
        }
        {
            std::lock_guard<std::mutex> g(mu_);
            fn_ = &fn;
            ntasks_ = ntasks;
            next_.store(0);
            active_ = n_ - 1;
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [this] { return active_ == 0; });
        fn_ = nullptr;
    }

  private:
    void work() {
        for (;;) {
            int64_t i = next_.fetch_add(1);
            if (i >= ntasks_) break;
            (*fn_)(i);
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return gen_ != seen; });
                seen = gen_;
                if (stop_) return;
            }
            work();
            {
                std::lock_guard<std::mutex> g(mu_);
                if (--active_ == 0) done_cv_.notify_all();
            }
        }
    }
    int n_;
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    uint64_t gen_ = 0;
    bool stop_ = false;
    int active_ = 0;
    const std::function<void(int64_t)>* fn_ = nullptr;
    int64_t ntasks_ = 0;
    std::atomic<int64_t> next_{0};
};

std::mutex g_pool_mu;
Pool* g_pool = nullptr;

Pool& pool_for(int nthreads) {
    int want = nthreads > 0 ? nthreads : qo_hardware_threads();
    std::lock_guard<std::mutex> g(g_pool_mu);
    if (!g_pool || g_pool->size() != want) {
        delete g_pool;
        g_pool = new Pool(want);
    }
    return *g_pool;
}

}  // namespace

extern "C" {

int qo_hardware_threads(void) {
    unsigned n = std::thread::hardware_concurrency();
    return n ? (int)n : 1;
}

// ---------------------------------------------------------------------------
// IEEE binary16 <-> binary32, round-to-nearest-even with subnormals: the
// behaviour of half 2.7.1's f16::from_f32 / f16::to_f32 (and of x86 F16C
// vcvtps2ph with RNE).
// ---------------------------------------------------------------------------
uint16_t qo_f16_from_f32(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));  // NaN
    if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);  // >= 2^16 (and inf): inf
    int e = (int)(ax >> 23) - 127;
    uint32_t m = ax & 0x7fffffu;
    if (e >= -14) {  // normal f16 (rounding may carry into the exponent, up to inf)
        uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
        uint32_t rem = m & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;
        return (uint16_t)(sign | h);
    }
    if (e < -25) return sign;  // below half the smallest subnormal: +-0
    m |= 0x800000u;
    int shift = -e - 1;  // 14 .. 24: units of 2^-24
    uint32_t h = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (h & 1u))) h += 1;
    return (uint16_t)(sign | h);
}

float qo_f32_from_f16(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {  // subnormal: m * 2^-24, renormalised
            int sh = 0;
            while (!(m & 0x400u)) {
                m <<= 1;
                ++sh;
            }
            m &= 0x3ffu;
            x = sign | ((uint32_t)(127 - 15 + 1 - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

// Arrays go through a 65536-entry table filled from qo_f32_from_f16 (every
// f16 value widens exactly, so the table is the function); large arrays are
// split over the worker pool.
void qo_f16_to_f32_array(const uint16_t* src, float* dst, int64_t n) {
    static const std::vector<float> table = [] {
        std::vector<float> t(65536);
        for (int i = 0; i < 65536; ++i) t[i] = qo_f32_from_f16((uint16_t)i);
        return t;
    }();
    const float* T = table.data();
    const int64_t blk = 1 << 20;
    if (n < 4 * blk) {
        for (int64_t i = 0; i < n; ++i) dst[i] = T[src[i]];
        return;
    }
    pool_for(0).run((n + blk - 1) / blk, [&](int64_t b) {
        const int64_t e = std::min(n, (b + 1) * blk);
        for (int64_t i = b * blk; i < e; ++i) dst[i] = T[src[i]];
    });
}

void qo_f32_to_f16_array(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = qo_f16_from_f32(src[i]);
}

// ---------------------------------------------------------------------------
// MRoPE tables.
// ---------------------------------------------------------------------------

// mrope.rs:5-41 build_dim_map.
int qo_build_dim_map(const int32_t* section, int nsec, int half, int interleaved, int32_t* out) {
    if (nsec <= 0 || half < 0) return -1;
    int len = 0;
    if (interleaved) {
        std::vector<int32_t> used(nsec, 0);
        while (len < half) {
            int before = len;
            for (int d = 0; d < nsec; ++d) {
                if (len >= half) break;
                if (used[d] < section[d]) {
                    out[len++] = d;
                    used[d] += 1;
                }
            }
            if (len == before) break;
        }
        // The Rust map may come out shorter than `half` when the quotas are
        // smaller; the callers then index past it and panic.  Report it.
        return len == half ? 0 : -1;
    }
    for (int d = 0; d < nsec; ++d) {
        for (int i = 0; i < section[d]; ++i) {
            if (len >= half) break;
            out[len++] = d;
        }
    }
    while (len < half) out[len++] = nsec - 1;
    return 0;
}

// mrope.rs:46-74 compute_mrope_cos_sin.  pos3 is [3][n] (pos[a][t]).
int qo_mrope_cos_sin(const int64_t* pos3, int n, int head_dim, double theta,
                     const int32_t* section, int nsec, int interleaved,
                     float* cos_out, float* sin_out) {
    if (head_dim <= 0 || head_dim % 2 || n < 0) return -1;
    const int half = head_dim / 2;
    std::vector<double> inv(half);
    for (int i = 0; i < half; ++i)
        inv[i] = 1.0 / std::pow(theta, 2.0 * (double)i / (double)head_dim);
    std::vector<int32_t> dm(half);
    if (qo_build_dim_map(section, nsec, half, interleaved, dm.data()) != 0) return -1;
    for (int d = 0; d < half; ++d)
        if (dm[d] < 0 || dm[d] > 2) return -1;  // pos has 3 axes
    for (int t = 0; t < n; ++t) {
        for (int j = 0; j < half; ++j) {
            double angle = (double)pos3[(int64_t)dm[j] * n + t] * inv[j];
            float c = (float)std::cos(angle);
            float s = (float)std::sin(angle);
            int64_t o = (int64_t)t * head_dim + j;
            cos_out[o] = c;
            sin_out[o] = s;
            cos_out[o + half] = c;
            sin_out[o + half] = s;
        }
    }
    return 0;
}

// text_positions (mrope.rs:77-80) -> compute_mrope_cos_sin -> f16
// (inference.rs:1038-1049).
int qo_text_rope_tables_f16(int rows, int head_dim, double theta,
                            const int32_t* section, int nsec, int interleaved,
                            uint16_t* cos_f16, uint16_t* sin_f16) {
    if (rows < 0) return -1;
    std::vector<int64_t> pos3((size_t)3 * rows);
    for (int a = 0; a < 3; ++a)
        for (int t = 0; t < rows; ++t) pos3[(size_t)a * rows + t] = t;
    std::vector<float> c((size_t)rows * head_dim), s((size_t)rows * head_dim);
    int rc = qo_mrope_cos_sin(pos3.data(), rows, head_dim, theta, section, nsec, interleaved,
                              c.data(), s.data());
    if (rc) return rc;
    qo_f32_to_f16_array(c.data(), cos_f16, (int64_t)c.size());
    qo_f32_to_f16_array(s.data(), sin_f16, (int64_t)s.size());
    return 0;
}

// ---------------------------------------------------------------------------
// cpu_decoder.rs:274-290 norm_rope_head.
// ---------------------------------------------------------------------------
void qo_norm_rope_head(const uint16_t* raw, const float* gain, const float* cos_row,
                       const float* sin_row, int hd, float eps, uint16_t* out) {
    const int half = hd / 2;
    float sum2 = 0.0f;
    for (int j = 0; j < hd; ++j) {
        float f = qo_f32_from_f16(raw[j]);
        sum2 += f * f;
    }
    float inv = 1.0f / std::sqrt(sum2 / (float)hd + eps);
    for (int j = 0; j < hd; ++j) {
        float xj = qo_f32_from_f16(raw[j]) * inv * gain[j];
        int pj = j < half ? j + half : j - half;
        float sign = j < half ? -1.0f : 1.0f;
        float xp = qo_f32_from_f16(raw[pj]) * inv * gain[pj];
        float c = cos_row[j], s = sin_row[j];
        out[j] = qo_f16_from_f32(xj * c + sign * xp * s);
    }
}

// ---------------------------------------------------------------------------
// cpu_decoder.rs:292-365 attention, one (row, q head) task per worker item.
// ---------------------------------------------------------------------------
int qo_attention(const qo_shape* sh, int cap, const uint16_t* q, int rows, int q0,
                 const float* k_cache, const float* v_cache, uint16_t* attn_out, int nthreads) {
    const int nqh = sh->nqh, nkvh = sh->nkvh, hd = sh->hd;
    if (nqh <= 0 || nkvh <= 0 || nqh % nkvh || hd <= 0 || hd % 4 || cap <= 0 || rows < 0 || q0 < 0)
        return -1;
    const float scale = 1.0f / std::sqrt((float)hd);
    const int rep = nqh / nkvh;
    const int64_t kv_stride = (int64_t)cap * hd;
    const int64_t row_elems = (int64_t)nqh * hd;
    Pool& pool = pool_for(nthreads);
    pool.run((int64_t)rows * nqh, [&](int64_t hi) {
        thread_local std::vector<float> scores, acc, qrow;
        if ((int)scores.size() < cap) scores.resize(cap);
        acc.resize(hd);
        qrow.resize(hd);
        const int r = (int)(hi / nqh), h = (int)(hi % nqh);
        const int pos = q0 + r;
        const int valid = std::min(pos + 1, cap);
        const uint16_t* qh = q + r * row_elems + (int64_t)h * hd;
        for (int d = 0; d < hd; ++d) qrow[d] = qo_f32_from_f16(qh[d]);
        const int kh = h / rep;
        const float* krow_all = k_cache + kh * kv_stride;
        const float* vrow_all = v_cache + kh * kv_stride;
        float best = -INFINITY;
        const int quads = hd / 4;
        for (int t = 0; t < valid; ++t) {
            const float* krow = krow_all + (int64_t)t * hd;
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
            for (int qd = 0; qd < quads; ++qd) {
                int j = qd * 4;
                a0 += qrow[j] * krow[j];
                a1 += qrow[j + 1] * krow[j + 1];
                a2 += qrow[j + 2] * krow[j + 2];
                a3 += qrow[j + 3] * krow[j + 3];
            }
            float dot = (a0 + a1) + (a2 + a3);
            float s = dot * scale;
            scores[t] = s;
            if (s > best) best = s;
        }
        float sum = 0.0f;
        for (int t = 0; t < valid; ++t) {
            scores[t] = std::exp(scores[t] - best);
            sum += scores[t];
        }
        float inv = 1.0f / sum;
        for (int j = 0; j < hd; ++j) acc[j] = 0.0f;
        for (int t = 0; t < valid; ++t) {
            float w = scores[t] * inv;
            const float* vrow = vrow_all + (int64_t)t * hd;
            for (int j = 0; j < hd; ++j) acc[j] += w * vrow[j];
        }
        uint16_t* out = attn_out + r * row_elems + (int64_t)h * hd;
        for (int j = 0; j < hd; ++j) out[j] = qo_f16_from_f32(acc[j]);
    });
    return 0;
}

// ---------------------------------------------------------------------------
// cpu_decoder.rs:398-423 -- stage (a) of forward() for one layer: q heads
// normed + roped into q_out, k heads normed + roped into k_cache[h][pos],
// v heads copied into v_cache[h][pos] (f32 holding f16 values).
// ---------------------------------------------------------------------------
int qo_qk_norm_rope_append(const qo_shape* sh, int cap, const uint16_t* qkv, int rows, int q0,
                           const uint16_t* q_gain, const uint16_t* k_gain,
                           const float* cos_tab, const float* sin_tab, int tab_rows,
                           float* k_cache, float* v_cache, uint16_t* q_out) {
    const int nqh = sh->nqh, nkvh = sh->nkvh, hd = sh->hd;
    if (nqh <= 0 || nkvh <= 0 || hd <= 0 || rows < 0 || q0 < 0) return -1;
    if (q0 + rows > sh->max_seq || q0 + rows > cap || q0 + rows > tab_rows) return -1;
    const int64_t q_dim = (int64_t)nqh * hd, kv_dim = (int64_t)nkvh * hd;
    const int64_t tot = q_dim + 2 * kv_dim;
    const int64_t kv_stride = (int64_t)cap * hd;
    std::vector<float> qn(hd), kn(hd);
    for (int j = 0; j < hd; ++j) {
        qn[j] = qo_f32_from_f16(q_gain[j]);
        kn[j] = qo_f32_from_f16(k_gain[j]);
    }
    std::vector<uint16_t> tmp(hd);
    for (int r = 0; r < rows; ++r) {
        const int pos = q0 + r;
        const uint16_t* row = qkv + r * tot;
        const float* c = cos_tab + (int64_t)pos * hd;
        const float* s = sin_tab + (int64_t)pos * hd;
        for (int h = 0; h < nqh; ++h)
            qo_norm_rope_head(row + h * hd, qn.data(), c, s, hd, sh->eps, q_out + r * q_dim + h * hd);
        for (int h = 0; h < nkvh; ++h) {
            qo_norm_rope_head(row + q_dim + h * hd, kn.data(), c, s, hd, sh->eps, tmp.data());
            float* kd = k_cache + h * kv_stride + (int64_t)pos * hd;
            for (int j = 0; j < hd; ++j) kd[j] = qo_f32_from_f16(tmp[j]);
            const uint16_t* vs = row + q_dim + kv_dim + h * hd;
            float* vd = v_cache + h * kv_stride + (int64_t)pos * hd;
            for (int j = 0; j < hd; ++j) vd[j] = qo_f32_from_f16(vs[j]);
        }
    }
    return 0;
}

// ---------------------------------------------------------------------------
// cpu_decoder.rs:398-427 -- the attention part of forward() for one layer.
// ---------------------------------------------------------------------------
int qo_layer_attn(const qo_shape* sh, int cap, const uint16_t* qkv, int rows, int q0,
                  const uint16_t* q_gain, const uint16_t* k_gain,
                  const float* cos_tab, const float* sin_tab, int tab_rows,
                  float* k_cache, float* v_cache, uint16_t* q_out, uint16_t* attn_out,
                  int nthreads) {
    int rc = qo_qk_norm_rope_append(sh, cap, qkv, rows, q0, q_gain, k_gain, cos_tab, sin_tab,
                                    tab_rows, k_cache, v_cache, q_out);
    if (rc) return rc;
    return qo_attention(sh, cap, q_out, rows, q0, k_cache, v_cache, attn_out, nthreads);
}

// cpu_decoder.rs:228 / decoder.rs:1610: grow-only, KV_STEP (256) granular,
// clamped to max_seq.
void qo_softmax_weights(const float* s, const float* m, int64_t n, float scale, float* out) {
    for (int64_t i = 0; i < n; ++i) {
        const float st = s[i] * scale;    // s = dot * scale
        const float best = m[i] * scale;  // the row's largest s
        out[i] = std::exp(st - best);     // (s - best).exp()
    }
}

int qo_kv_target_cap(int need, int cap, int max_seq) {
    const int step = 256;
    int64_t t = ((int64_t)need + step - 1) / step * step;
    t = std::min<int64_t>(t, max_seq);
    t = std::max<int64_t>(t, cap);
    return (int)t;
}

// ---------------------------------------------------------------------------
// Seeded inputs.  SplitMix64 (Steele, Lea & Flood 2014); uniforms in (0, 1)
// from the top 53 bits plus half an ulp; Box-Muller pairs in f64.
// ---------------------------------------------------------------------------
uint64_t qo_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double unit_open(uint64_t* st) {
    return ((double)(qo_splitmix64(st) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

void qo_fill_normal_f16(uint64_t* state, int64_t n, double mean, double std, uint16_t* out) {
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = unit_open(state), u2 = unit_open(state);
        double r = std::sqrt(-2.0 * std::log(u1));
        double z0 = r * std::cos(two_pi * u2), z1 = r * std::sin(two_pi * u2);
        out[i] = qo_f16_from_f32((float)(mean + std * z0));
        if (i + 1 < n) out[i + 1] = qo_f16_from_f32((float)(mean + std * z1));
    }
}

int32_t qo_uniform_int(uint64_t* state, int32_t lo, int32_t hi) {
    uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    return (int32_t)((int64_t)lo + (int64_t)(qo_splitmix64(state) % span));
}

// ===========================================================================
// The whole text decoder for one sequence: CpuTextDecoder (cpu_decoder.rs).
// Test infrastructure for the end-to-end greedy check: the attention path
// under test sits inside this layer sequence on the GPU side.
// ===========================================================================
}  // extern "C"

namespace {

// Mat (cpu_decoder.rs:11-27) holds f16 checkpoint weights widened to f32.
// Here the f16 rows are read in place (borrowed from the caller) and widened
// four at a time with vcvtph2ps, which is exact, so the products are the same
// f32 products.  [rows][cols].
struct Mat {
    const uint16_t* w = nullptr;
    int rows = 0, cols = 0;
    void load(const uint16_t* p, int r, int c) {
        w = p;
        rows = r;
        cols = c;
    }
    // dot_transposed (cpu_decoder.rs:64-100) for one row x (f32 values of f16):
    // four strided partial sums a[k % 4] (one SSE lane each: a separate
    // multiply and add per element, as in Rust), then (a0 + a1) + (a2 + a3),
    // then the tail.  Output blocks of 64 rows run as pool tasks, as the
    // reference's par_chunks.
    void dot(const float* x, float* acc, Pool& pool) const {
        const int OB = 64;
        const int64_t nblk = (rows + OB - 1) / OB;
        pool.run(nblk, [&](int64_t bi) {
            const int o1 = std::min<int>(rows, (int)(bi + 1) * OB);
            for (int o = (int)bi * OB; o < o1; ++o) {
                const uint16_t* wr = w + (size_t)o * cols;
                __m128 a = _mm_setzero_ps();
                const int quads = cols / 4;
                for (int q = 0; q < quads; ++q) {
                    const __m128 wv = _mm_cvtph_ps(_mm_loadl_epi64((const __m128i*)(wr + 4 * q)));
                    a = _mm_add_ps(a, _mm_mul_ps(wv, _mm_loadu_ps(x + 4 * q)));
                }
                float a4[4];
                _mm_storeu_ps(a4, a);
                float s = (a4[0] + a4[1]) + (a4[2] + a4[3]);
                for (int k = quads * 4; k < cols; ++k) s += qo_f32_from_f16(wr[k]) * x[k];
                acc[o] = s;
            }
        });
    }
};

struct DecLayer {
    std::vector<float> iln, pln, qn, kn;
    std::vector<uint16_t> qn16, kn16;
    Mat q, k, v, o, gate, up, down;
};

struct Decoder {
    qo_dec_cfg cfg;
    int cap = 0;
    const uint16_t* embed = nullptr;  // f16, as the reference keeps it (borrowed)
    std::vector<float> norm_w;
    std::vector<DecLayer> layers;
    std::vector<float> cos, sin;  // f32 values of the f16 tables
    int tab_rows = 0;
    std::vector<float> k_cache, v_cache;  // [layer][nkvh][cap][hd]
    int pos = 0;
    uint32_t last_token = 0;
};

std::vector<float> widen(const uint16_t* p, int64_t n) {
    std::vector<float> v(n);
    qo_f16_to_f32_array(p, v.data(), n);
    return v;
}

// rms_norm_row (cpu_decoder.rs:261-272): sequential sum of squares,
// inv = 1 / sqrt(sum2 / n + eps), out = f16(x * inv * w).
void rms_norm_row(const uint16_t* x, const float* w, int n, float eps, uint16_t* out) {
    float sum2 = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float f = qo_f32_from_f16(x[i]);
        sum2 += f * f;
    }
    const float inv = 1.0f / std::sqrt(sum2 / (float)n + eps);
    for (int i = 0; i < n; ++i) out[i] = qo_f16_from_f32(qo_f32_from_f16(x[i]) * inv * w[i]);
}

// forward (cpu_decoder.rs:367-456) for rows q0..q0+rows-1 of hidden state x
// ([rows][hs] f16, updated in place).  Rows >= 2 use the reference's gemm crate
// there (gemm 0.18.2, summation order not restated); here every row takes the
// one-row order of dot_transposed.
void forward(Decoder& D, std::vector<uint16_t>& x, int q0, int rows, Pool& pool) {
    const qo_dec_cfg& c = D.cfg;
    const int hs = c.hs, nqh = c.nqh, nkvh = c.nkvh, hd = c.hd, inter = c.inter;
    const int q_dim = nqh * hd, kv_dim = nkvh * hd, tot = q_dim + 2 * kv_dim;
    const int64_t layer_kv = (int64_t)nkvh * D.cap * hd;
    std::vector<uint16_t> normed((size_t)rows * hs), qkv((size_t)rows * tot), qout((size_t)rows * q_dim),
        attn((size_t)rows * q_dim), gate16((size_t)inter), up16((size_t)inter);
    std::vector<float> xf(std::max(hs, std::max(q_dim, inter))), acc(std::max(tot, std::max(hs, inter)));
    qo_shape sh{nqh, nkvh, hd, c.max_seq, c.eps};
    for (int li = 0; li < c.layers; ++li) {
        DecLayer& L = D.layers[li];
        // input norm + q/k/v projections (383-394), f16 after each projection
        for (int r = 0; r < rows; ++r) {
            rms_norm_row(&x[(size_t)r * hs], L.iln.data(), hs, c.eps, &normed[(size_t)r * hs]);
            qo_f16_to_f32_array(&normed[(size_t)r * hs], xf.data(), hs);
            uint16_t* row = &qkv[(size_t)r * tot];
            L.q.dot(xf.data(), acc.data(), pool);
            for (int i = 0; i < q_dim; ++i) row[i] = qo_f16_from_f32(acc[i]);
            L.k.dot(xf.data(), acc.data(), pool);
            for (int i = 0; i < kv_dim; ++i) row[q_dim + i] = qo_f16_from_f32(acc[i]);
            L.v.dot(xf.data(), acc.data(), pool);
            for (int i = 0; i < kv_dim; ++i) row[q_dim + kv_dim + i] = qo_f16_from_f32(acc[i]);
        }
        // q/k norm + RoPE, KV append, attention (396-427)
        if (qo_layer_attn(&sh, D.cap, qkv.data(), rows, q0, L.qn16.data(), L.kn16.data(), D.cos.data(),
                          D.sin.data(), D.tab_rows, D.k_cache.data() + li * layer_kv,
                          D.v_cache.data() + li * layer_kv, qout.data(), attn.data(), 0))
            return;
        for (int r = 0; r < rows; ++r) {
            uint16_t* xr = &x[(size_t)r * hs];
            // o_proj + residual (429): x = f16(x + acc)
            qo_f16_to_f32_array(&attn[(size_t)r * q_dim], xf.data(), q_dim);
            L.o.dot(xf.data(), acc.data(), pool);
            for (int i = 0; i < hs; ++i) xr[i] = qo_f16_from_f32(qo_f32_from_f16(xr[i]) + acc[i]);
            // post-attention norm, gate/up, SiLU * up, down + residual (433-447)
            rms_norm_row(xr, L.pln.data(), hs, c.eps, &normed[(size_t)r * hs]);
            qo_f16_to_f32_array(&normed[(size_t)r * hs], xf.data(), hs);
            L.gate.dot(xf.data(), acc.data(), pool);
            for (int i = 0; i < inter; ++i) gate16[i] = qo_f16_from_f32(acc[i]);
            L.up.dot(xf.data(), acc.data(), pool);
            for (int i = 0; i < inter; ++i) up16[i] = qo_f16_from_f32(acc[i]);
            for (int i = 0; i < inter; ++i) {
                const float g = qo_f32_from_f16(gate16[i]);
                const float silu = g / (1.0f + std::exp(-g));
                gate16[i] = qo_f16_from_f32(silu * qo_f32_from_f16(up16[i]));
            }
            qo_f16_to_f32_array(gate16.data(), xf.data(), inter);
            L.down.dot(xf.data(), acc.data(), pool);
            for (int i = 0; i < hs; ++i) xr[i] = qo_f16_from_f32(qo_f32_from_f16(xr[i]) + acc[i]);
        }
    }
}

// final_norm_logits + argmax (cpu_decoder.rs:458-482): logits against the
// tied embedding, sequential f32 sums; the first maximum wins.
int final_logits_argmax(Decoder& D, const uint16_t* x_last, float* logits_out, Pool& pool) {
    const int hs = D.cfg.hs, vocab = D.cfg.vocab;
    std::vector<uint16_t> normed(hs);
    rms_norm_row(x_last, D.norm_w.data(), hs, D.cfg.eps, normed.data());
    std::vector<float> nf(hs), logits(vocab);
    qo_f16_to_f32_array(normed.data(), nf.data(), hs);
    const int64_t blk = 256;
    pool.run((vocab + blk - 1) / blk, [&](int64_t bi) {
        const int t1 = std::min<int>(vocab, (int)(bi + 1) * blk);
        for (int t = (int)bi * blk; t < t1; ++t) {
            const uint16_t* row = D.embed + (size_t)t * hs;
            float a = 0.0f;
            int i = 0;
            for (; i + 4 <= hs; i += 4) {  // widen 4 at a time, add in order
                float w4[4];
                _mm_storeu_ps(w4, _mm_cvtph_ps(_mm_loadl_epi64((const __m128i*)(row + i))));
                a += w4[0] * nf[i];
                a += w4[1] * nf[i + 1];
                a += w4[2] * nf[i + 2];
                a += w4[3] * nf[i + 3];
            }
            for (; i < hs; ++i) a += qo_f32_from_f16(row[i]) * nf[i];
            logits[t] = a;
        }
    });
    int best = 0;
    for (int t = 0; t < vocab; ++t)
        if (logits[t] > logits[best]) best = t;
    if (logits_out) std::memcpy(logits_out, logits.data(), sizeof(float) * vocab);
    return best;
}

}  // namespace

extern "C" {

void* qo_dec_create(const qo_dec_cfg* cfg, const uint16_t* embed, const uint16_t* final_norm,
                    const uint16_t* const* layer_ptrs, int cap) {
    if (!cfg || !embed || !final_norm || !layer_ptrs) return nullptr;
    const qo_dec_cfg& c = *cfg;
    if (c.hs <= 0 || c.nqh <= 0 || c.nkvh <= 0 || c.nqh % c.nkvh || c.hd <= 0 || c.hd % 4 ||
        c.inter <= 0 || c.layers <= 0 || c.vocab <= 0 || cap <= 0 || cap > c.max_seq)
        return nullptr;
    Decoder* D = new Decoder();
    D->cfg = c;
    D->cap = cap;
    D->embed = embed;
    D->norm_w = widen(final_norm, c.hs);
    D->layers.resize(c.layers);
    const int q_dim = c.nqh * c.hd, kv_dim = c.nkvh * c.hd;
    for (int l = 0; l < c.layers; ++l) {
        const uint16_t* const* p = layer_ptrs + 11 * l;
        DecLayer& L = D->layers[l];
        L.iln = widen(p[0], c.hs);
        L.pln = widen(p[1], c.hs);
        L.qn16.assign(p[2], p[2] + c.hd);
        L.kn16.assign(p[3], p[3] + c.hd);
        L.q.load(p[4], q_dim, c.hs);
        L.k.load(p[5], kv_dim, c.hs);
        L.v.load(p[6], kv_dim, c.hs);
        L.o.load(p[7], c.hs, q_dim);
        L.gate.load(p[8], c.inter, c.hs);
        L.up.load(p[9], c.inter, c.hs);
        L.down.load(p[10], c.hs, c.inter);
    }
    const size_t kvn = (size_t)c.layers * c.nkvh * cap * c.hd;
    D->k_cache.assign(kvn, 0.0f);
    D->v_cache.assign(kvn, 0.0f);
    return D;
}

void qo_dec_destroy(void* d) { delete (Decoder*)d; }

int qo_dec_set_rope(void* d, const uint16_t* cos_f16, const uint16_t* sin_f16, int rows) {
    Decoder* D = (Decoder*)d;
    if (!D || !cos_f16 || !sin_f16 || rows <= 0) return -1;
    D->cos = widen(cos_f16, (int64_t)rows * D->cfg.hd);
    D->sin = widen(sin_f16, (int64_t)rows * D->cfg.hd);
    D->tab_rows = rows;
    return 0;
}

int qo_dec_prefill(void* d, const uint16_t* hidden, int s, int kv_start, float* logits) {
    Decoder* D = (Decoder*)d;
    if (!D || !hidden || s <= 0 || kv_start < 0 || kv_start + s > D->cap || kv_start + s > D->tab_rows)
        return -1;
    const int hs = D->cfg.hs;
    std::vector<uint16_t> x(hidden, hidden + (size_t)s * hs);
    Pool& pool = pool_for(0);
    forward(*D, x, kv_start, s, pool);
    D->pos = kv_start + s;
    const int tok = final_logits_argmax(*D, &x[(size_t)(s - 1) * hs], logits, pool);
    D->last_token = (uint32_t)tok;
    return tok;
}

int qo_dec_step(void* d, float* logits) {
    Decoder* D = (Decoder*)d;
    if (!D || D->pos >= D->cap || D->pos >= D->tab_rows) return -1;
    const int hs = D->cfg.hs;
    std::vector<uint16_t> x(D->embed + (size_t)D->last_token * hs,
                            D->embed + (size_t)(D->last_token + 1) * hs);
    Pool& pool = pool_for(0);
    forward(*D, x, D->pos, 1, pool);
    D->pos += 1;
    const int tok = final_logits_argmax(*D, x.data(), logits, pool);
    D->last_token = (uint32_t)tok;
    return tok;
}

int qo_dec_pos(void* d) { return d ? ((Decoder*)d)->pos : -1; }

}  // extern "C"
