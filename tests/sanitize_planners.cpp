// sanitize_planners.cpp -- host sanitizer driver for the library's launch
// planners (qasr_plan_decode, qasr_plan_prefill).  Built by
// `python tests/sanitize_planners.py`: every source's host code
// with AddressSanitizer and UndefinedBehaviorSanitizer (device code as
// usual), linked into one executable with this file.  No device is touched:
// the planners are host code.  It drives them over random batches, the edge
// cases of every argument, the environment knobs and the refusals, and
// checks the plans' invariants; the sanitizers check every access and every
// integer operation on the way.  Exit status 0 when everything holds.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "qasr_attn.h"

namespace {

int failures = 0;

void check(bool ok, const char* what, long long a = 0, long long b = 0) {
    if (ok) return;
    std::fprintf(stderr, "FAIL: %s (%lld, %lld)\n", what, a, b);
    ++failures;
}

uint64_t rng_state = 0x5A417E5EEDull;
uint64_t next_u64() {  // SplitMix64
    uint64_t z = (rng_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
int uniform(int lo, int hi) { return lo + (int)(next_u64() % (uint64_t)(hi - lo + 1)); }

constexpr int kMaxPos = 1 << 24;

// Every key of every entry in exactly one granule, granules whole
// workgroup passes and at most 32 per entry, runs within the granules,
// bases add up.
void decode_case(const std::vector<int32_t>& lens, int nkvh, int cus) {
    const int n = (int)lens.size();
    std::vector<int32_t> gran(n + 1, -1), run(n + 1, -1), base(n + 2, -1);
    const int rc = qasr_plan_decode(n, lens.data(), nkvh, cus, gran.data(), run.data(), base.data());
    check(rc == QASR_OK, "qasr_plan_decode refused a valid batch", n, rc);
    if (rc != QASR_OK) return;
    check(base[0] == 0, "wg_base[0]", base[0]);
    for (int b = 0; b < n; ++b) {
        const int64_t g = gran[b], L = lens[b], r = run[b];
        check(g >= 256 && g % 256 == 0, "granule not whole pass pairs", b, g);
        if (g <= 0) continue;
        const int64_t ngr = (L + g - 1) / g;
        check((ngr - 1) * g < L && L <= ngr * g, "granules do not tile the entry", L, g);
        check(ngr <= 32, "granules per entry", ngr);
        check(r >= 1 && r <= ngr && r <= 8 && r * g <= (1 << 22) + g, "granules per workgroup", b, r);
        if (r <= 0) continue;
        check((int64_t)base[b + 1] - base[b] == nkvh * ((ngr + r - 1) / r), "wg_base step", b,
              base[b + 1] - base[b]);
    }
    check(gran[n] == -1 && run[n] == -1 && base[n + 1] == -1, "wrote past the outputs");
}

// Row blocks cover the rows; every row block's key tiles are covered by its
// splits; at most 65 bases written.
void prefill_case(int rows, int kv_start, int nkvh) {
    int32_t rpb = -1, nrb = -1, tps = -1;
    std::vector<int32_t> sp(67, -1);
    const int rc = qasr_plan_prefill(rows, kv_start, nkvh, &rpb, &nrb, &tps, sp.data());
    check(rc == QASR_OK, "qasr_plan_prefill refused valid rows", rows, kv_start);
    if (rc != QASR_OK) return;
    check(rpb == 64 || rpb == 32 || rpb == 16, "rows per block", rpb);
    check(nrb >= 1 && nrb <= 64 && (int64_t)nrb * rpb >= rows && (int64_t)(nrb - 1) * rpb < rows,
          "row blocks", nrb, rows);
    check(tps >= 1, "tiles per split", tps);
    check(sp[0] == 0, "sp_base[0]", sp[0]);
    for (int rb = 0; rb < nrb && rb < 64; ++rb) {
        const int64_t kend = (int64_t)kv_start + std::min<int64_t>((int64_t)(rb + 1) * rpb, rows);
        const int64_t tiles = (kend + 127) / 128;
        const int64_t splits = (int64_t)sp[rb + 1] - sp[rb];
        check(splits >= 1 && splits * tps >= tiles && (splits - 1) * tps < tiles, "splits of a row block", rb,
              splits);
        check(rpb == 64 || splits == 1, "a 32- or 16-row block split", rb, splits);
    }
    check(sp[66] == -1, "wrote past 65 bases");
}

void refusals() {
    int32_t lens[65], gran[66], run[66], base[66];
    for (int i = 0; i < 65; ++i) lens[i] = 100;
    check(qasr_plan_decode(0, lens, 8, 256, gran, run, base) == QASR_EINVAL, "batch 0 accepted");
    check(qasr_plan_decode(65, lens, 8, 256, gran, run, base) == QASR_EINVAL, "batch 65 accepted");
    check(qasr_plan_decode(1, lens, 0, 256, gran, run, base) == QASR_EINVAL, "nkvh 0 accepted");
    check(qasr_plan_decode(1, lens, 65, 256, gran, run, base) == QASR_EINVAL, "nkvh 65 accepted");
    check(qasr_plan_decode(1, lens, 8, 0, gran, run, base) == QASR_EINVAL, "cus 0 accepted");
    check(qasr_plan_decode(1, nullptr, 8, 256, gran, run, base) == QASR_EINVAL, "null lens accepted");
    lens[0] = 0;
    check(qasr_plan_decode(1, lens, 8, 256, gran, run, base) == QASR_EINVAL, "empty entry accepted");
    lens[0] = kMaxPos + 1;
    check(qasr_plan_decode(1, lens, 8, 256, gran, run, base) == QASR_EINVAL, "2^24 + 1 keys accepted");
    lens[0] = 2147483647;
    check(qasr_plan_decode(1, lens, 8, 256, gran, run, base) == QASR_EINVAL, "INT_MAX keys accepted");
    int32_t rpb, nrb, tps, sp[65];
    check(qasr_plan_prefill(0, 0, 8, &rpb, &nrb, &tps, sp) == QASR_EINVAL, "0 rows accepted");
    check(qasr_plan_prefill(4097, 0, 8, &rpb, &nrb, &tps, sp) == QASR_EINVAL, "4097 rows accepted");
    check(qasr_plan_prefill(16, -1, 8, &rpb, &nrb, &tps, sp) == QASR_EINVAL, "kv_start -1 accepted");
    check(qasr_plan_prefill(16, kMaxPos + 1, 8, &rpb, &nrb, &tps, sp) == QASR_EINVAL, "kv_start 2^24 + 1");
    check(qasr_plan_prefill(16, 2147483647, 8, &rpb, &nrb, &tps, sp) == QASR_EINVAL, "kv_start INT_MAX");
    check(qasr_plan_prefill(16, 0, 8, nullptr, &nrb, &tps, sp) == QASR_EINVAL, "null output accepted");
}

}  // namespace

int main() {
    refusals();
    const char* knobs[][2] = {{nullptr, nullptr},
                              {"QASR_DECODE_WGS", "1"},
                              {"QASR_DECODE_WGS", "4096"},
                              {"QASR_DECODE_GRANULE", "32"},
                              {"QASR_DECODE_GRANULE", "100000"},
                              {"QASR_DECODE_MAX_GRANULES", "1"},
                              {"QASR_DECODE_MAX_GRANULES", "100000"},
                              {"QASR_DECODE_WGS", "-5"},
                              {"QASR_PREFILL_TPS", "1"},
                              {"QASR_PREFILL_TPS", "7"},
                              {"QASR_PREFILL_TPS", "100000"}};
    int cases = 0;
    for (const auto& k : knobs) {
        if (k[0]) setenv(k[0], k[1], 1);
        // decode: random batches, then the edges of each argument
        for (int it = 0; it < 400; ++it) {
            const int n = uniform(1, 64);
            const int hi = it % 4 == 0 ? kMaxPos : it % 4 == 1 ? 16384 : it % 4 == 2 ? 600 : 40;
            std::vector<int32_t> lens(n);
            for (auto& L : lens) L = uniform(1, hi);
            decode_case(lens, uniform(1, 64), uniform(1, 1024));
            ++cases;
        }
        for (int n : {1, 2, 63, 64})
            for (int L : {1, 31, 32, 33, 8193, kMaxPos - 1, kMaxPos})
                for (int nkvh : {1, 8, 64})
                    for (int cus : {1, 256, 1 << 20}) {
                        decode_case(std::vector<int32_t>(n, L), nkvh, cus);
                        ++cases;
                    }
        // prefill: random rows / starts, then the edges
        for (int it = 0; it < 400; ++it) {
            prefill_case(uniform(1, 4096), uniform(0, it % 2 ? kMaxPos : 9000), uniform(1, 64));
            ++cases;
        }
        for (int rows : {1, 31, 32, 33, 63, 64, 65, 420, 512, 4095, 4096})
            for (int ks : {0, 1, 127, 128, 420, 7680, kMaxPos - 4096, kMaxPos})
                for (int nkvh : {1, 8, 64}) {
                    prefill_case(rows, ks, nkvh);
                    ++cases;
                }
        if (k[0]) unsetenv(k[0]);
    }
    std::printf("planner sanitizer driver: %d cases, %d failures\n", cases, failures);
    return failures ? 1 : 0;
}
