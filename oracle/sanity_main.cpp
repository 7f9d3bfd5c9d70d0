// sanity_main.cpp -- host AddressSanitizer / UBSan driver for the oracle
// (`make -C oracle sanity`).  TEST INFRASTRUCTURE: exercises every entry
// point of oracle.h on small shapes, including the edge sizes (one key,
// cap-limited attention, chunked prefill), so out-of-bounds indexing in the
// restatement shows up on the CPU.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "oracle.h"

static int g_fail = 0;
#define CHECK(c)                                                    \
    do {                                                            \
        if (!(c)) {                                                 \
            std::fprintf(stderr, "FAIL %s:%d %s\n", __FILE__, __LINE__, #c); \
            ++g_fail;                                               \
        }                                                           \
    } while (0)

int main() {
    uint64_t st = 0x51A50000ull;
    // conversions, exhaustive round trip of finite f16 values
    for (int h = 0; h < 65536; ++h) {
        const float f = qo_f32_from_f16((uint16_t)h);
        if (std::isfinite(f)) CHECK(qo_f16_from_f32(f) == (uint16_t)h || f == 0.0f);
    }
    // tables
    const int rows = 64, hd = 128;
    std::vector<uint16_t> cs(rows * hd), sn(rows * hd);
    const int32_t sec[3] = {24, 20, 20};
    CHECK(qo_text_rope_tables_f16(rows, hd, 1e6, sec, 3, 1, cs.data(), sn.data()) == 0);
    std::vector<float> cf(rows * hd), sf(rows * hd);
    qo_f16_to_f32_array(cs.data(), cf.data(), rows * hd);
    qo_f16_to_f32_array(sn.data(), sf.data(), rows * hd);
    // layer attention, full and chunked, at cap-limited sizes
    qo_shape sh{4, 2, hd, rows, 1e-6f};
    const int tot = (4 + 2 * 2) * hd, cap = 48;
    std::vector<uint16_t> qkv(cap * tot), gq(hd), gk(hd), q(cap * 4 * hd), o(cap * 4 * hd);
    qo_fill_normal_f16(&st, (int64_t)qkv.size(), 0.0, 1.0, qkv.data());
    qo_fill_normal_f16(&st, hd, 1.0, 0.1, gq.data());
    qo_fill_normal_f16(&st, hd, 1.0, 0.1, gk.data());
    std::vector<float> kc(2 * cap * hd), vc(2 * cap * hd);
    CHECK(qo_layer_attn(&sh, cap, qkv.data(), 1, 0, gq.data(), gk.data(), cf.data(), sf.data(), rows,
                        kc.data(), vc.data(), q.data(), o.data(), 2) == 0);
    CHECK(qo_layer_attn(&sh, cap, qkv.data(), cap - 1, 1, gq.data(), gk.data(), cf.data(), sf.data(),
                        rows, kc.data(), vc.data(), q.data(), o.data(), 3) == 0);
    CHECK(qo_layer_attn(&sh, cap, qkv.data(), 2, cap - 1, gq.data(), gk.data(), cf.data(), sf.data(),
                        rows, kc.data(), vc.data(), q.data(), o.data(), 2) != 0);  // past cap
    // whole decoder, tiny shape: prefill, chunked prefill, steps
    const qo_dec_cfg c{32, 4, 2, 16, 48, 2, 40, 32, 1e-6f};
    std::vector<std::vector<uint16_t>> store;
    auto tensor = [&](int64_t n, double mean, double sd) {
        store.emplace_back(n);
        qo_fill_normal_f16(&st, n, mean, sd, store.back().data());
        return store.back().data();
    };
    store.reserve(64);
    const uint16_t* embed = tensor((int64_t)c.vocab * c.hs, 0.0, 0.1);
    const uint16_t* norm = tensor(c.hs, 1.0, 0.1);
    std::vector<const uint16_t*> lp;
    for (int l = 0; l < c.layers; ++l) {
        const int qd = c.nqh * c.hd, kd = c.nkvh * c.hd;
        lp.push_back(tensor(c.hs, 1.0, 0.1));
        lp.push_back(tensor(c.hs, 1.0, 0.1));
        lp.push_back(tensor(c.hd, 1.0, 0.1));
        lp.push_back(tensor(c.hd, 1.0, 0.1));
        lp.push_back(tensor((int64_t)qd * c.hs, 0.0, 0.2));
        lp.push_back(tensor((int64_t)kd * c.hs, 0.0, 0.2));
        lp.push_back(tensor((int64_t)kd * c.hs, 0.0, 0.2));
        lp.push_back(tensor((int64_t)c.hs * qd, 0.0, 0.5));
        lp.push_back(tensor((int64_t)c.inter * c.hs, 0.0, 0.2));
        lp.push_back(tensor((int64_t)c.inter * c.hs, 0.0, 0.2));
        lp.push_back(tensor((int64_t)c.hs * c.inter, 0.0, 0.5));
    }
    std::vector<uint16_t> tcs(32 * 16), tsn(32 * 16);
    const int32_t sec16[3] = {3, 3, 2};
    CHECK(qo_text_rope_tables_f16(32, 16, 1e6, sec16, 3, 1, tcs.data(), tsn.data()) == 0);
    void* d = qo_dec_create(&c, embed, norm, lp.data(), 32);
    CHECK(d != nullptr);
    CHECK(qo_dec_set_rope(d, tcs.data(), tsn.data(), 32) == 0);
    std::vector<uint16_t> hid(10 * c.hs);
    qo_fill_normal_f16(&st, (int64_t)hid.size(), 0.0, 1.0, hid.data());
    std::vector<float> logits(c.vocab);
    CHECK(qo_dec_prefill(d, hid.data(), 4, 0, logits.data()) >= 0);
    CHECK(qo_dec_prefill(d, hid.data() + 4 * c.hs, 6, 4, nullptr) >= 0);
    for (int i = 0; i < 22; ++i) CHECK(qo_dec_step(d, logits.data()) >= 0);
    CHECK(qo_dec_pos(d) == 32);
    CHECK(qo_dec_step(d, nullptr) < 0);  // cap reached: refused, no write past the caches
    qo_dec_destroy(d);
    std::printf("oracle sanity: %s\n", g_fail ? "FAILED" : "ok");
    return g_fail ? 1 : 0;
}
