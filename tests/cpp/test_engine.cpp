// test_engine.cpp -- tests of the C++ API (serving-engine_amd/engine/*.h)
// written the way the reference's own C++ tests exercise engine::cuda and
// engine::KVCache (reference tests/test_kv_cache.cpp:43-200,
// tests/test_attention.cpp:34-291): random shapes, fp16-rounded inputs,
// GPU result against a CPU reference.  Here the CPU reference is the oracle
// (oracle/kvhp_oracle.h), and the tolerance is |g - r| <= 2e-3 + 1e-2 |r|
// per element plus max |g - r| <= 2e-3, stricter than the reference's 3e-3
// / 3.5e-3 max-abs.  Copies are checked bit for bit.
//
//   test_engine --cpu   cases that need no GPU (fp16 conversion, host
//                       validation errors, page bookkeeping)
//   test_engine --gpu   every case
// Exit status 0 when every check passed.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "forward_gpu.h"
#include "hip_utils.h"
#include "half.h"
#include "kernels.h"
#include "kv_cache.h"
#include "kv_view.h"
#include "kvhp_oracle.h"
#include "llama_runner.h"

using namespace engine;

namespace {

int g_checks = 0;
int g_failures = 0;
std::string g_case;

#define EXPECT(cond, ...)                                                          \
    do {                                                                           \
        ++g_checks;                                                                \
        if (!(cond)) {                                                             \
            ++g_failures;                                                          \
            if (g_failures < 40) {                                                 \
                std::printf("  FAIL [%s] %s:%d: %s -- ", g_case.c_str(), __FILE__, \
                            __LINE__, #cond);                                      \
                std::printf(__VA_ARGS__);                                          \
                std::printf("\n");                                                 \
            }                                                                      \
        }                                                                          \
    } while (0)

std::vector<half> random_half(std::mt19937& rng, size_t n, float lo, float hi) {
    std::uniform_real_distribution<float> dist(lo, hi);
    std::vector<half> v(n);
    for (auto& x : v) x = float_to_half(dist(rng));
    return v;
}

std::vector<float> to_float(const std::vector<half>& h) {
    std::vector<float> f(h.size());
    for (size_t i = 0; i < h.size(); ++i) f[i] = half_to_float(h[i]);
    return f;
}

template <typename T>
DeviceBuffer<T> upload(const std::vector<T>& v) {
    DeviceBuffer<T> d(v.size());
    d.copy_from_host(v.data(), v.size());
    return d;
}

template <typename T>
std::vector<T> download(const DeviceBuffer<T>& d) {
    std::vector<T> v(d.size());
    d.copy_to_host(v.data(), v.size());
    return v;
}

// Compares fp16 GPU output with an fp32 reference; returns the max abs diff.
float check_close(const std::vector<half>& got, const std::vector<float>& ref, const char* what) {
    float worst = 0.f;
    size_t bad = 0, first_bad = 0;
    for (size_t i = 0; i < ref.size(); ++i) {
        const float g = half_to_float(got[i]);
        const float d = std::fabs(g - ref[i]);
        if (!(d <= 2e-3f + 1e-2f * std::fabs(ref[i]))) {
            if (!bad) first_bad = i;
            ++bad;
        }
        if (!(d <= worst)) worst = d;
    }
    EXPECT(bad == 0 && worst <= 2e-3f, "%s: %zu elements out of tolerance (first %zu), max abs %.3g",
           what, bad, first_bad, worst);
    return worst;
}

bool bits_equal(const std::vector<half>& a, const std::vector<half>& b) {
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(half)) == 0;
}

// ------------------------------------------------------------- CPU cases --

void case_half_conversion() {
    // every binary16 pattern survives half -> float -> half (NaNs stay NaN)
    // and agrees with the oracle's independent conversion
    for (uint32_t b = 0; b < 65536; ++b) {
        const half h{(uint16_t)b};
        const float f = half_to_float(h);
        const float fo = kvo_f16_to_f32((uint16_t)b);
        const bool nan = ((b >> 10) & 0x1f) == 0x1f && (b & 0x3ff);
        if (nan) {
            EXPECT(std::isnan(f), "pattern %04x", b);
            continue;
        }
        EXPECT(std::memcmp(&f, &fo, 4) == 0, "pattern %04x -> %g vs oracle %g", b, f, fo);
        EXPECT(float_to_half(f).bits == b, "pattern %04x round trip", b);
    }
    // float -> half rounding (ties to even, subnormals, overflow) against the
    // oracle over random bit patterns and the halfway points of every
    // adjacent pair of finite halves
    std::mt19937 rng(11);
    for (int i = 0; i < 2000000; ++i) {
        uint32_t x = rng();
        float f;
        std::memcpy(&f, &x, 4);
        if (std::isnan(f)) continue;
        EXPECT(float_to_half(f).bits == kvo_f32_to_f16(f), "float bits %08x", x);
    }
    for (uint32_t b = 0; b < 0x7bff; ++b) {
        const double lo = half_to_float(half{(uint16_t)b});
        const double hi = half_to_float(half{(uint16_t)(b + 1)});
        const float mid = (float)((lo + hi) / 2);  // exact in float
        EXPECT(float_to_half(mid).bits == kvo_f32_to_f16(mid), "tie above %04x", b);
        EXPECT(float_to_half(-mid).bits == kvo_f32_to_f16(-mid), "tie below -%04x", b);
    }
}

void case_host_validation() {
    // Hq not a multiple of Hkv, and head_dim beyond 256, are rejected before
    // any device work, as a thrown std::runtime_error
    half dummy[8] = {};
    hip::KVView v{dummy, 0, 0, 8, 1};
    int lens = 1;
    bool threw = false;
    try {
        hip::decode_gqa_split(dummy, v, v, &lens, dummy, 1, 6, 4, 64, 16);
    } catch (const std::runtime_error& e) {
        threw = std::string(e.what()).find("num_q_heads") != std::string::npos;
    }
    EXPECT(threw, "decode_gqa_split accepted Hq=6, Hkv=4");
    threw = false;
    try {
        hip::flash_prefill_gqa(dummy, dummy, dummy, dummy, 4, 4, 4, 512, 1);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    EXPECT(threw, "flash_prefill_gqa accepted head_dim=512");
    // empty work is a no-op, as in the reference (kv_cache.cu:50)
    bool ok = true;
    try {
        hip::append_kv_cache(dummy, dummy, dummy, dummy, 0, 0, 1, 16, 8);
        hip::decode_gqa(dummy, dummy, dummy, dummy, 0, 4, 4, 16, 8);
    } catch (...) {
        ok = false;
    }
    EXPECT(ok, "empty work threw");
    // the reference-signature split buffer holds 8 splits' worth of partials
    EXPECT(hip::decode_split_buffer_floats(3, 14, 64) == (size_t)8 * 3 * 14 * 66, "size");
    EXPECT(hip::decode_workspace_bytes(3, 14, 2, 64, 600, 8) <=
               hip::decode_split_buffer_floats(3, 14, 64) * sizeof(float),
           "8-split workspace larger than the split buffer");
}

void case_kv_view_get_ptr() {
    // reference kv_view.h:24-30: data + b*stride_b + h*stride_h + s*stride_s
    // (+ d*stride_d), here with stride_d != 1 and a non-literal d
    std::vector<half> buf(8192);
    const half* base = buf.data();
    const hip::KVView v{base, 1000, 200, 12, 3};
    for (int b = 0; b < 3; ++b)
        for (int h = 0; h < 2; ++h)
            for (int s = 0; s < 5; ++s) {
                EXPECT(v.get_ptr(b, h, s) == base + b * 1000 + h * 200 + s * 12, "(%d,%d,%d)", b, h, s);
                for (int d = 0; d < 4; ++d)
                    EXPECT(v.get_ptr(b, h, s, d) == base + b * 1000 + h * 200 + s * 12 + d * 3,
                           "(%d,%d,%d,%d)", b, h, s, d);
            }
    // paged view: page table [2 sequences][3 pages] of a pool of 8 pages,
    // D = 4; the table is host memory here, so get_ptr and get_ptr_host agree
    const std::vector<int32_t> table = {5, 2, 7, 1, 0, 3};
    const hip::KVView p = hip::paged_view(base, 8, 4, table.data(), 3);
    for (int b = 0; b < 2; ++b)
        for (int h = 0; h < 2; ++h)
            for (int s = 0; s < 48; s += 5)
                for (int d = 0; d < 4; ++d) {
                    const half* want = base + h * (8 * 16 * 4) +
                                       ((int64_t)table[b * 3 + s / 16] * 16 + s % 16) * 4 + d;
                    EXPECT(p.get_ptr(b, h, s, d) == want, "paged (%d,%d,%d,%d)", b, h, s, d);
                    EXPECT(p.get_ptr_host(b, h, s, d, table.data()) == want, "paged host");
                }
    EXPECT(v.get_ptr_host(1, 1, 2, 3, nullptr) == v.get_ptr(1, 1, 2, 3), "strided host form");
}

// ------------------------------------------------------------- GPU cases --

void case_kv_cache_layout() {
    // pointer arithmetic of reference kv_cache.h:34-53
    KVCache c(3, 4, 64, 40);
    const size_t per = (size_t)4 * 40 * 64;
    EXPECT(c.get_layer_ptr(0, 0) == c.raw_data(), "layer 0 K");
    EXPECT(c.get_layer_ptr(1, 1) == c.raw_data() + 3 * per, "layer 1 V");
    EXPECT(c.get_head_ptr(2, 1, 3) == c.raw_data() + 5 * per + 3 * 40 * 64, "head ptr");
    EXPECT(c.current_seq_len() == 0, "fresh length");
    c.set_current_seq_len(7);
    EXPECT(c.current_seq_len() == 7, "length");
    // allocate() zeroes the cache
    std::vector<half> all((size_t)3 * 2 * per);
    HIP_CHECK(hipMemcpy(all.data(), c.raw_data(), all.size() * 2, hipMemcpyDeviceToHost));
    bool zero = true;
    for (auto h : all) zero &= h.bits == 0;
    EXPECT(zero, "cache not zeroed");
}

void case_append_kv_cache() {
    // 25 random shapes (reference test_kv_cache.cpp:43-97), bit-exact
    std::mt19937 rng(1101);
    for (int it = 0; it < 25; ++it) {
        const int T = it == 0 ? 1 : 1 + (int)(rng() % 37);
        const int start = it == 0 ? 0 : (int)(rng() % 50);
        const int hkv = 1 + (int)(rng() % 4);
        // some shapes run past max_seq: those positions must be dropped
        const int max_seq = start + T + (int)(rng() % 30) - (it % 5 == 4 ? T / 2 : 0);
        const int d = 16 * (1 + (int)(rng() % 8));
        auto ks = random_half(rng, (size_t)T * hkv * d, -2, 2);
        auto vs = random_half(rng, (size_t)T * hkv * d, -2, 2);
        const size_t csz = (size_t)hkv * max_seq * d;
        auto dk = upload(ks), dv = upload(vs);
        DeviceBuffer<half> ck(csz), cv(csz);
        ck.zero();
        cv.zero();
        hip::append_kv_cache(dk.data(), dv.data(), ck.data(), cv.data(), T, start, hkv, max_seq, d);
        HIP_CHECK(hipDeviceSynchronize());
        std::vector<uint16_t> rk(csz, 0), rv(csz, 0);
        kvo_append_kv(reinterpret_cast<const uint16_t*>(ks.data()),
                      reinterpret_cast<const uint16_t*>(vs.data()), rk.data(), rv.data(), T, start,
                      hkv, max_seq, d);
        auto gk = download(ck), gv = download(cv);
        EXPECT(std::memcmp(gk.data(), rk.data(), csz * 2) == 0, "K shape %d (T=%d start=%d hkv=%d max_seq=%d d=%d)", it, T, start, hkv, max_seq, d);
        EXPECT(std::memcmp(gv.data(), rv.data(), csz * 2) == 0, "V shape %d", it);
    }
}

void case_decode_gqa() {
    // 25 random shapes over a head-major cache (test_kv_cache.cpp:99-200)
    std::mt19937 rng(1102);
    for (int it = 0; it < 25; ++it) {
        const int L = it == 0 ? 1 : 1 + (int)(rng() % 300);
        const int max_seq = L + (int)(rng() % 32);
        const int hkv = 1 + (int)(rng() % 3);
        const int g = 1 + (int)(rng() % 5);
        const int hq = hkv * g;
        const int d = it % 3 == 0 ? 128 : 16 * (1 + (int)(rng() % 4));
        auto q = random_half(rng, (size_t)hq * d, -1, 1);
        auto k = random_half(rng, (size_t)hkv * max_seq * d, -1, 1);
        auto v = random_half(rng, (size_t)hkv * max_seq * d, -1, 1);
        auto dq = upload(q), dk = upload(k), dv = upload(v);
        DeviceBuffer<half> out((size_t)hq * d);
        hip::decode_gqa(dq.data(), dk.data(), dv.data(), out.data(), L, hq, hkv, max_seq, d);
        HIP_CHECK(hipDeviceSynchronize());
        std::vector<float> ref((size_t)hq * d);
        const int32_t len = L;
        kvo_decode_attention(to_float(q).data(), to_float(k).data(), to_float(v).data(), &len,
                             ref.data(), 1, hq, hkv, d, max_seq, 1);
        char what[96];
        std::snprintf(what, sizeof what, "decode_gqa shape %d (L=%d hq=%d hkv=%d d=%d)", it, L, hq, hkv, d);
        check_close(download(out), ref, what);
    }
}

void case_decode_gqa_split() {
    // 25 random batched shapes (test_attention.cpp:34-183): group size 7
    // every third shape, lengths 1, 17, 513 and random; with the reference's
    // 8-split buffer and with the library workspace
    std::mt19937 rng(1701);
    for (int it = 0; it < 25; ++it) {
        const int b = it % 4 == 0 ? 1 : 1 + (int)(rng() % 3);
        const int hkv = 2;
        const int g = it % 3 == 0 ? 7 : 1 + (int)(rng() % 7);
        const int hq = hkv * g;
        const int d = it % 2 ? 64 : 128;
        std::vector<int> lens(b);
        int max_seq = 0;
        for (int i = 0; i < b; ++i) {
            lens[i] = it == 0 ? 1 : it == 1 ? 17 : it == 2 ? 513 : 1 + (int)(rng() % 2000);
            max_seq = std::max(max_seq, lens[i]);
        }
        auto q = random_half(rng, (size_t)b * hq * d, -1, 1);
        auto k = random_half(rng, (size_t)b * hkv * max_seq * d, -1, 1);
        auto v = random_half(rng, (size_t)b * hkv * max_seq * d, -1, 1);
        auto dq = upload(q), dk = upload(k), dv = upload(v);
        auto dl = upload(lens);
        DeviceBuffer<half> out((size_t)b * hq * d), out2((size_t)b * hq * d);
        DeviceBuffer<float> split(hip::decode_split_buffer_floats(b, hq, d));
        const auto kv = hip::contiguous_view(dk.data(), hkv, max_seq, d);
        const auto vv = hip::contiguous_view(dv.data(), hkv, max_seq, d);
        hip::decode_gqa_split(dq.data(), kv, vv, dl.data(), out.data(), b, hq, hkv, d, max_seq,
                              split.data());
        hip::decode_gqa_split(dq.data(), kv, vv, dl.data(), out2.data(), b, hq, hkv, d, max_seq);
        HIP_CHECK(hipDeviceSynchronize());
        std::vector<float> ref((size_t)b * hq * d);
        kvo_decode_attention(to_float(q).data(), to_float(k).data(), to_float(v).data(),
                             lens.data(), ref.data(), b, hq, hkv, d, max_seq, 4);
        char what[96];
        std::snprintf(what, sizeof what, "split_buffer shape %d (b=%d g=%d d=%d L0=%d)", it, b, g, d, lens[0]);
        check_close(download(out), ref, what);
        std::snprintf(what, sizeof what, "library workspace shape %d", it);
        check_close(download(out2), ref, what);
    }
}

void case_flash_prefill_gqa() {
    // 25 random shapes (test_attention.cpp:188-291): S = 1, 15, 17, 65 and
    // random, group size 7 every third shape, D = 64 and 128, batch 1..2
    std::mt19937 rng(1702);
    for (int it = 0; it < 25; ++it) {
        const int b = it % 5 == 4 ? 2 : 1;
        const int hkv = 2;
        const int g = it % 3 == 0 ? 7 : 1 + (int)(rng() % 7);
        const int hq = hkv * g;
        const int d = it % 2 ? 64 : 128;
        const int S = it == 0 ? 1 : it == 1 ? 15 : it == 2 ? 17 : it == 3 ? 65 : 1 + (int)(rng() % 300);
        auto q = random_half(rng, (size_t)b * S * hq * d, -1, 1);
        auto k = random_half(rng, (size_t)b * S * hkv * d, -1, 1);
        auto v = random_half(rng, (size_t)b * S * hkv * d, -1, 1);
        auto dq = upload(q), dk = upload(k), dv = upload(v);
        DeviceBuffer<half> out(q.size());
        hip::flash_prefill_gqa(dq.data(), dk.data(), dv.data(), out.data(), S, hq, hkv, d, b);
        HIP_CHECK(hipDeviceSynchronize());
        const auto qf = to_float(q), kf = to_float(k), vf = to_float(v);
        std::vector<float> ref(q.size());
        for (int s = 0; s < b; ++s)
            kvo_causal_gqa_rows(qf.data() + (size_t)s * S * hq * d, kf.data() + (size_t)s * S * hkv * d,
                                vf.data() + (size_t)s * S * hkv * d, ref.data() + (size_t)s * S * hq * d,
                                S, hq, hkv, d, 0, S, 4);
        char what[96];
        std::snprintf(what, sizeof what, "flash_prefill shape %d (b=%d S=%d g=%d d=%d)", it, b, S, g, d);
        check_close(download(out), ref, what);
    }
}

void case_causal_gqa() {
    // the naive reference op is routed to the flash kernel: same results
    std::mt19937 rng(1703);
    const int S = 77, hq = 8, hkv = 2, d = 48;  // D outside the MFMA path
    auto q = random_half(rng, (size_t)S * hq * d, -1, 1);
    auto k = random_half(rng, (size_t)S * hkv * d, -1, 1);
    auto v = random_half(rng, (size_t)S * hkv * d, -1, 1);
    auto dq = upload(q), dk = upload(k), dv = upload(v);
    DeviceBuffer<half> out(q.size());
    hip::causal_gqa(dq.data(), dk.data(), dv.data(), out.data(), S, hq, hkv, d);
    HIP_CHECK(hipDeviceSynchronize());
    std::vector<float> ref(q.size());
    kvo_causal_gqa(to_float(q).data(), to_float(k).data(), to_float(v).data(), ref.data(), S, hq, hkv, d);
    check_close(download(out), ref, "causal_gqa");
}

void case_paged_identity_equals_kvcache() {
    // One sequence whose pages are taken in order from a fresh pool has the
    // identity block table, so the paged pool and KVCache's head-major block
    // must hold the same bytes after the same appends.
    std::mt19937 rng(1704);
    const int layers = 2, hkv = 4, d = 64, max_seq = 96;
    KVCache flat(layers, hkv, d, max_seq);
    PagedKVCache paged(layers, hkv, d, max_seq / 16, 1, max_seq / 16);
    const int slot = paged.add_sequence();
    EXPECT(slot == 0, "first slot %d", slot);
    int pos = 0;
    for (int chunk : {37, 1, 1, 20, 5}) {
        paged.begin_prefill(1, chunk);
        paged.sync();
        for (int l = 0; l < layers; ++l) {
            auto ks = random_half(rng, (size_t)chunk * hkv * d, -2, 2);
            auto vs = random_half(rng, (size_t)chunk * hkv * d, -2, 2);
            auto dk = upload(ks), dv = upload(vs);
            hip::append_kv_cache(dk.data(), dv.data(), flat.get_layer_ptr(l, 0),
                                 flat.get_layer_ptr(l, 1), chunk, pos, hkv, max_seq, d);
            paged.append(l, dk.data(), dv.data(), 1, chunk);
            HIP_CHECK(hipDeviceSynchronize());
        }
        pos += chunk;
    }
    EXPECT(paged.seq_len(0) == pos, "length %d vs %d", paged.seq_len(0), pos);
    for (int i = 0; i < paged.pages_used(0); ++i)
        EXPECT(paged.host_block_table(0)[i] == i, "page %d -> %d", i, paged.host_block_table(0)[i]);
    for (int l = 0; l < layers; ++l)
        for (int kv = 0; kv < 2; ++kv) {
            std::vector<half> a((size_t)hkv * max_seq * d), p(a.size());
            HIP_CHECK(hipMemcpy(a.data(), flat.get_layer_ptr(l, kv), a.size() * 2, hipMemcpyDeviceToHost));
            HIP_CHECK(hipMemcpy(p.data(), paged.get_layer_ptr(l, kv), p.size() * 2, hipMemcpyDeviceToHost));
            EXPECT(bits_equal(a, p), "layer %d %s differs", l, kv ? "V" : "K");
        }
}

void case_paged_serving_steps() {
    // Runner flow over PagedKVCache: prefill three sequences (K/V written to
    // pages by the prefill kernel), then decode steps with "bump, then write
    // at num_tokens - 1"; every step's attention is checked against the oracle
    // over the full history, and a freed sequence's pages are reused.
    std::mt19937 rng(1705);
    const int hq = 8, hkv = 2, d = 128, B = 3, steps = 4;
    const int prompt[B] = {40, 17, 90};
    PagedKVCache cache(1, hkv, d, 64, B, 16);
    std::vector<std::vector<half>> hist_k(B), hist_v(B);  // [t][hkv][d] per sequence
    for (int s = 0; s < B; ++s) {
        EXPECT(cache.add_sequence() == s, "slot %d", s);
        const int S = prompt[s];
        auto q = random_half(rng, (size_t)S * hq * d, -1, 1);
        hist_k[s] = random_half(rng, (size_t)S * hkv * d, -1, 1);
        hist_v[s] = random_half(rng, (size_t)S * hkv * d, -1, 1);
        cache.reserve(s, S);
        cache.set_seq_len(s, S);
        cache.sync();
        auto dq = upload(q), dk = upload(hist_k[s]), dv = upload(hist_v[s]);
        DeviceBuffer<half> out(q.size());
        // one sequence's own block-table row
        hip::flash_prefill_gqa_paged(dq.data(), dk.data(), dv.data(), out.data(), S, hq, hkv, d, 1,
                                     cache.get_layer_ptr(0, 0), cache.get_layer_ptr(0, 1),
                                     cache.block_tables() + (size_t)s * cache.max_pages_per_seq(),
                                     cache.max_pages_per_seq(), cache.num_pages());
        HIP_CHECK(hipDeviceSynchronize());
        std::vector<float> ref(q.size());
        kvo_causal_gqa_rows(to_float(q).data(), to_float(hist_k[s]).data(), to_float(hist_v[s]).data(),
                            ref.data(), S, hq, hkv, d, 0, S, 4);
        check_close(download(out), ref, "paged prefill");
    }
    auto run_steps = [&](int nsteps) {
        for (int st = 0; st < nsteps; ++st) {
            cache.begin_decode_step(B);
            cache.sync();
            auto q = random_half(rng, (size_t)B * hq * d, -1, 1);
            auto kn = random_half(rng, (size_t)B * hkv * d, -1, 1);
            auto vn = random_half(rng, (size_t)B * hkv * d, -1, 1);
            auto dq = upload(q), dk = upload(kn), dv = upload(vn);
            DeviceBuffer<half> out(q.size());
            int max_len = 0;
            for (int s = 0; s < B; ++s) max_len = std::max(max_len, cache.seq_len(s));
            if (st % 2 == 0) {  // separate calls, then the fused step, alternately
                cache.append(0, dk.data(), dv.data(), B, 1);
                cache.decode(0, dq.data(), out.data(), B, hq, max_len);
            } else {
                cache.append_decode(0, dk.data(), dv.data(), dq.data(), out.data(), B, hq, max_len);
            }
            HIP_CHECK(hipDeviceSynchronize());
            // oracle over the contiguous history [B][hkv][max_len][d]
            std::vector<float> kc((size_t)B * hkv * max_len * d, 0.f), vc(kc.size(), 0.f);
            std::vector<int32_t> lens(B);
            for (int s = 0; s < B; ++s) {
                hist_k[s].insert(hist_k[s].end(), kn.begin() + (size_t)s * hkv * d, kn.begin() + (size_t)(s + 1) * hkv * d);
                hist_v[s].insert(hist_v[s].end(), vn.begin() + (size_t)s * hkv * d, vn.begin() + (size_t)(s + 1) * hkv * d);
                lens[s] = cache.seq_len(s);
                EXPECT((size_t)lens[s] * hkv * d == hist_k[s].size(), "history length of %d", s);
                for (int t = 0; t < lens[s]; ++t)
                    for (int h = 0; h < hkv; ++h)
                        for (int i = 0; i < d; ++i) {
                            const size_t dst = (((size_t)s * hkv + h) * max_len + t) * d + i;
                            const size_t src = ((size_t)t * hkv + h) * d + i;
                            kc[dst] = half_to_float(hist_k[s][src]);
                            vc[dst] = half_to_float(hist_v[s][src]);
                        }
            }
            std::vector<float> ref(q.size());
            kvo_decode_attention(to_float(q).data(), kc.data(), vc.data(), lens.data(), ref.data(),
                                 B, hq, hkv, d, max_len, 4);
            char what[64];
            std::snprintf(what, sizeof what, "paged decode step (lens %d,%d,%d)", lens[0], lens[1], lens[2]);
            check_close(download(out), ref, what);
        }
    };
    run_steps(steps);
    // sequence 1 finishes; a new one takes its slot and reuses its pages
    const int freed = cache.pages_used(1);
    const int before = cache.free_page_count();
    cache.release(1);
    EXPECT(cache.free_page_count() == before + freed, "pages not returned");
    EXPECT(cache.add_sequence() == 1, "slot reuse");
    hist_k[1].clear();
    hist_v[1].clear();
    {
        const int S = 33;
        hist_k[1] = random_half(rng, (size_t)S * hkv * d, -1, 1);
        hist_v[1] = random_half(rng, (size_t)S * hkv * d, -1, 1);
        cache.set_seq_len(1, S);
        cache.sync();
        std::vector<int32_t> zero_pos(B, 0);
        auto dk = upload(hist_k[1]), dv = upload(hist_v[1]);
        DeviceBuffer<int32_t> pos = upload(zero_pos);
        hip::paged_append_kv(dk.data(), dv.data(), cache.get_layer_ptr(0, 0), cache.get_layer_ptr(0, 1),
                             cache.block_tables() + (size_t)cache.max_pages_per_seq(),
                             cache.max_pages_per_seq(), pos.data(), 1, S, hkv, d, cache.num_pages());
        HIP_CHECK(hipDeviceSynchronize());
    }
    run_steps(2);
    // the gather of every sequence reproduces its history bit for bit
    int max_len = 0;
    std::vector<int32_t> lens(B);
    for (int s = 0; s < B; ++s) max_len = std::max(max_len, lens[s] = cache.seq_len(s));
    DeviceBuffer<half> gk((size_t)B * hkv * max_len * d), gv(gk.size());
    DeviceBuffer<int32_t> dl = upload(lens);
    hip::paged_gather_kv(cache.get_layer_ptr(0, 0), cache.get_layer_ptr(0, 1), cache.block_tables(),
                         cache.max_pages_per_seq(), dl.data(), B, hkv, d, cache.num_pages(), max_len,
                         gk.data(), gv.data());
    HIP_CHECK(hipDeviceSynchronize());
    auto hk = download(gk);
    bool same = true;
    for (int s = 0; s < B; ++s)
        for (int t = 0; t < lens[s]; ++t)
            for (int h = 0; h < hkv; ++h)
                same &= std::memcmp(&hk[(((size_t)s * hkv + h) * max_len + t) * d],
                                    &hist_k[s][((size_t)t * hkv + h) * d], d * 2) == 0;
    EXPECT(same, "gathered K differs from the appended history");
}

void case_paged_cache_rejects() {
    // Host-side contract of PagedKVCache: out-of-range batches, layers and
    // slots, negative lengths, page exhaustion and a full batch all throw
    // before any device work.
    PagedKVCache cache(2, 2, 64, 4, 2, 3);   // 4 pages, 2 slots, 3 pages per sequence
    auto throws = [](auto&& f) {
        try {
            f();
        } catch (const std::exception&) {
            return true;
        }
        return false;
    };
    half dummy[8] = {};
    EXPECT(throws([&] { cache.begin_decode_step(3); }), "batch 3 of 2 accepted");
    EXPECT(throws([&] { cache.begin_prefill(-1, 4); }), "negative batch accepted");
    EXPECT(throws([&] { cache.begin_prefill(1, -4); }), "negative token count accepted");
    EXPECT(throws([&] { cache.set_seq_len(0, -1); }), "negative length accepted");
    EXPECT(throws([&] { cache.set_seq_len(2, 1); }), "slot 2 of 2 accepted");
    EXPECT(throws([&] { cache.decode(2, dummy, dummy, 1, 4, 16); }), "layer 2 of 2 accepted");
    EXPECT(throws([&] { cache.append(0, dummy, dummy, 3, 1); }), "append batch 3 accepted");
    EXPECT(throws([&] { cache.reserve(0, 4 * 16); }), "more pages than max_pages_per_seq");
    EXPECT(cache.add_sequence() == 0 && cache.add_sequence() == 1, "slots");
    EXPECT(throws([&] { cache.add_sequence(); }), "third sequence in a batch of 2");
    cache.reserve(0, 3 * 16);
    EXPECT(throws([&] { cache.reserve(1, 2 * 16); }), "reserved past the pool (4 pages)");
    EXPECT(cache.free_page_count() == 1, "a failed reserve took pages");
}

void case_paged_prefix_sharing() {
    // Prefix sharing (docs/runner_interface.md:30-33, 51): sequence B shares
    // A's two full prompt pages, recomputes its whole prompt in "share" mode
    // with K/V that differ on the shared part, and the prefill's page writes
    // through write_block_tables() leave A's pages untouched.  Decode steps
    // then write only private pages; a decode write into a shared page
    // throws before any slot changes; pages return to the free list when the
    // last holder releases them.
    std::mt19937 rng(2207);
    const int hq = 4, hkv = 2, d = 64, SA = 40, SB = 45;
    PagedKVCache cache(1, hkv, d, 16, 3, 8);
    const int mp = cache.max_pages_per_seq();
    auto gather = [&](int slot, int len) {
        DeviceBuffer<half> gk((size_t)hkv * len * d), gv(gk.size());
        std::vector<int32_t> l1 = {len};
        DeviceBuffer<int32_t> dl = upload(l1);
        hip::paged_gather_kv(cache.get_layer_ptr(0, 0), cache.get_layer_ptr(0, 1),
                             cache.block_tables() + (size_t)slot * mp, mp, dl.data(), 1, hkv, d,
                             cache.num_pages(), len, gk.data(), gv.data());
        HIP_CHECK(hipDeviceSynchronize());
        return std::make_pair(download(gk), download(gv));
    };
    // token-major [T][hkv][d] -> head-major [hkv][T][d]
    auto head_major = [&](const std::vector<half>& x, int T) {
        std::vector<half> y(x.size());
        for (int t = 0; t < T; ++t)
            for (int h = 0; h < hkv; ++h)
                std::memcpy(&y[((size_t)h * T + t) * d], &x[((size_t)t * hkv + h) * d], d * 2);
        return y;
    };
    auto prefill = [&](int slot, int S, const std::vector<half>& k, const std::vector<half>& v) {
        auto q = random_half(rng, (size_t)S * hq * d, -1, 1);
        auto dq = upload(q), dk = upload(k), dv = upload(v);
        DeviceBuffer<half> out(q.size());
        hip::flash_prefill_gqa_paged(dq.data(), dk.data(), dv.data(), out.data(), S, hq, hkv, d, 1,
                                     cache.get_layer_ptr(0, 0), cache.get_layer_ptr(0, 1),
                                     cache.write_block_tables() + (size_t)slot * mp, mp,
                                     cache.num_pages());
        HIP_CHECK(hipDeviceSynchronize());
        std::vector<float> ref(q.size());
        kvo_causal_gqa_rows(to_float(q).data(), to_float(k).data(), to_float(v).data(), ref.data(), S,
                            hq, hkv, d, 0, S, 4);
        check_close(download(out), ref, "prefill");
    };

    const int a = cache.add_sequence();
    auto ka = random_half(rng, (size_t)SA * hkv * d, -1, 1), va = random_half(rng, ka.size(), -1, 1);
    cache.set_seq_len(a, SA);
    cache.sync();
    prefill(a, SA, ka, va);

    const int b = cache.add_sequence();
    EXPECT(cache.share_prefix(b, a, SA) == 32, "shared token count");
    EXPECT(cache.seq_len(b) == 32 && cache.pages_used(b) == 2, "B after share: %d tokens, %d pages",
           cache.seq_len(b), cache.pages_used(b));
    for (int i = 0; i < 2; ++i) {
        EXPECT(cache.host_block_table(b)[i] == cache.host_block_table(a)[i], "page %d not shared", i);
        EXPECT(cache.page_refs(cache.host_block_table(a)[i]) == 2, "refs of shared page %d", i);
    }
    EXPECT(cache.page_refs(cache.host_block_table(a)[2]) == 1, "A's partial page shared");
    // "share" mode: B recomputes all 45 prompt tokens; its K/V on the shared
    // 32 differ from A's, so any write into a shared page would show.
    auto kb = random_half(rng, (size_t)SB * hkv * d, -1, 1), vb = random_half(rng, kb.size(), -1, 1);
    cache.set_seq_len(b, SB);
    cache.sync();
    prefill(b, SB, kb, vb);
    auto ga = gather(a, SA);
    EXPECT(bits_equal(ga.first, head_major(ka, SA)) && bits_equal(ga.second, head_major(va, SA)),
           "A's pages changed by B's prefill");
    // B's cache: A's K/V on the shared pages, its own after them
    std::vector<half> hb_k(kb), hb_v(vb);
    std::copy(ka.begin(), ka.begin() + (size_t)32 * hkv * d, hb_k.begin());
    std::copy(va.begin(), va.begin() + (size_t)32 * hkv * d, hb_v.begin());
    auto gb = gather(b, SB);
    EXPECT(bits_equal(gb.first, head_major(hb_k, SB)) && bits_equal(gb.second, head_major(hb_v, SB)),
           "B's cache is not A's shared prefix + B's own suffix");

    // two decode steps for both: writes land on private pages only
    std::vector<half> hist_k[2] = {ka, hb_k}, hist_v[2] = {va, hb_v};
    for (int st = 0; st < 2; ++st) {
        cache.begin_decode_step(2);
        cache.sync();
        auto q = random_half(rng, (size_t)2 * hq * d, -1, 1);
        auto kn = random_half(rng, (size_t)2 * hkv * d, -1, 1), vn = random_half(rng, kn.size(), -1, 1);
        auto dq = upload(q), dk = upload(kn), dv = upload(vn);
        DeviceBuffer<half> out(q.size());
        const int max_len = std::max(cache.seq_len(a), cache.seq_len(b));
        cache.append_decode(0, dk.data(), dv.data(), dq.data(), out.data(), 2, hq, max_len);
        HIP_CHECK(hipDeviceSynchronize());
        std::vector<float> kc((size_t)2 * hkv * max_len * d, 0.f), vc(kc.size(), 0.f);
        std::vector<int32_t> lens = {cache.seq_len(a), cache.seq_len(b)};
        for (int s = 0; s < 2; ++s) {
            hist_k[s].insert(hist_k[s].end(), kn.begin() + (size_t)s * hkv * d, kn.begin() + (size_t)(s + 1) * hkv * d);
            hist_v[s].insert(hist_v[s].end(), vn.begin() + (size_t)s * hkv * d, vn.begin() + (size_t)(s + 1) * hkv * d);
            for (int t = 0; t < lens[s]; ++t)
                for (int h = 0; h < hkv; ++h)
                    for (int i = 0; i < d; ++i) {
                        kc[(((size_t)s * hkv + h) * max_len + t) * d + i] = half_to_float(hist_k[s][((size_t)t * hkv + h) * d + i]);
                        vc[(((size_t)s * hkv + h) * max_len + t) * d + i] = half_to_float(hist_v[s][((size_t)t * hkv + h) * d + i]);
                    }
        }
        std::vector<float> ref(q.size());
        kvo_decode_attention(to_float(q).data(), kc.data(), vc.data(), lens.data(), ref.data(), 2, hq,
                             hkv, d, max_len, 4);
        check_close(download(out), ref, "decode over a shared prefix");
    }
    ga = gather(a, SA + 2);
    gb = gather(b, SB + 2);
    EXPECT(bits_equal(ga.first, head_major(hist_k[0], SA + 2)), "A's history after decode");
    EXPECT(bits_equal(gb.first, head_major(hist_k[1], SB + 2)) &&
               bits_equal(gb.second, head_major(hist_v[1], SB + 2)),
           "B's history after decode");

    // C shares B's prefix, then is cut back into a shared page: its decode
    // write would mutate a shared page, so the step throws and changes nothing
    const int c = cache.add_sequence();
    EXPECT(cache.share_prefix(c, b, 40) == 32, "C's shared count");
    cache.set_seq_len(c, 20);
    const int len_a = cache.seq_len(a), free_before = cache.free_page_count();
    bool threw = false;
    try {
        cache.begin_decode_step(3);
    } catch (const std::logic_error&) {
        threw = true;
    }
    EXPECT(threw, "decode write into a shared page accepted");
    EXPECT(cache.seq_len(a) == len_a && cache.seq_len(c) == 20 && cache.free_page_count() == free_before,
           "a rejected step changed the cache");
    EXPECT(cache.page_refs(cache.host_block_table(b)[0]) == 3, "refs with three holders");

    // release: a page is freed only by its last holder
    const int shared0 = cache.host_block_table(a)[0];
    const int priv_a = cache.pages_used(a) - 2;
    cache.release(a);
    EXPECT(cache.free_page_count() == free_before + priv_a, "A's release freed %d pages, expected %d",
           cache.free_page_count() - free_before, priv_a);
    EXPECT(cache.page_refs(shared0) == 2, "refs after A's release");
    cache.release(c);
    EXPECT(cache.page_refs(shared0) == 1 && cache.free_page_count() == free_before + priv_a,
           "C's release freed pages B still holds");
    cache.release(b);
    EXPECT(cache.page_refs(shared0) == 0 && cache.free_page_count() == cache.num_pages(),
           "every page free after the last release");
    EXPECT(cache.add_sequence() == 0, "slot reuse after release");
    EXPECT(cache.add_sequence() == 1, "slot reuse after release");
    bool bad_share = false;
    try {
        cache.share_prefix(1, 0, 16);   // source holds 0 tokens
    } catch (const std::out_of_range&) {
        bad_share = true;
    }
    EXPECT(bad_share, "prefix longer than the source accepted");
}

void case_llama_runner_paged() {
    // LlamaRunner over a PagedKVCache (Runner.prefill / decode_step,
    // docs/runner_interface.md:18-53): three sequences, the third sharing the
    // first's two full prompt pages and forwarding only its suffix ("full"
    // prefix mode), then batched decode steps with an idle fourth slot.  Each
    // slot against a batch-1 model of the same seed fed the same tokens:
    // prefill logits bit-identical (within 2% for the cached-prefix one);
    // decode logits within 2% of the logit scale, a differing greedy token
    // only at a near-tie (top-1 / top-2 margin of the batch-1 logits below
    // 0.05).
    const kvhp_llama_config c = {1024, 256, 2, 4, 2, 64, 512, 1e-5f, 10000.f, 0};
    const uint64_t seed = 31;
    const int V = c.vocab_size;
    LlamaRunner runner(c, seed, 64);
    PagedKVCache cache(c.num_layers, c.num_kv_heads, c.head_dim, 32, 4, 8);
    std::mt19937 rng(77);
    std::uniform_int_distribution<int> tokd(0, V - 1);
    std::vector<std::vector<int32_t>> prompts(3);
    prompts[0].resize(35);
    prompts[1].resize(19);
    for (int s = 0; s < 2; ++s)
        for (auto& t : prompts[s]) t = tokd(rng);
    prompts[2].assign(prompts[0].begin(), prompts[0].begin() + 32);
    for (int i = 0; i < 7; ++i) prompts[2].push_back(tokd(rng));
    void* ref[3] = {};
    for (auto& r : ref) KVHP_CHECK(kvhp_llama_create(&c, seed, 64, &r));
    auto compare = [&](const float* got, const std::vector<float>& want, int tok, int want_tok,
                       const char* what) {
        float scale = 1.f, diff = 0.f, top1 = -INFINITY, top2 = -INFINITY;
        for (int i = 0; i < V; ++i) {
            scale = std::max(scale, std::fabs(want[i]));
            diff = std::max(diff, std::fabs(got[i] - want[i]));
            if (want[i] > top1) {
                top2 = top1;
                top1 = want[i];
            } else if (want[i] > top2) {
                top2 = want[i];
            }
        }
        EXPECT(diff < 0.02f * scale, "%s: max |logit diff| %.4f, scale %.2f", what, diff, scale);
        EXPECT(tok == want_tok || top1 - top2 < 0.05f, "%s: token %d != %d, margin %.4f", what, tok,
               want_tok, top1 - top2);
    };
    std::vector<int32_t> last(4, 0);
    for (int s = 0; s < 3; ++s) {
        EXPECT(cache.add_sequence() == s, "slot %d", s);
        int cached = 0;
        if (s == 2) EXPECT((cached = cache.share_prefix(2, 0, 35)) == 32, "shared prefix");
        cache.set_seq_len(s, (int)prompts[s].size());
        std::vector<float> lg, rl(V);
        // slot 2 forwards only its uncached suffix ("full" prefix mode)
        const int tok = runner.prefill(cache, s, prompts[s], &lg, nullptr, cached);
        int32_t rt = -1;
        KVHP_CHECK(kvhp_llama_prefill(ref[s], prompts[s].data(), (int)prompts[s].size(), rl.data(), &rt));
        if (cached == 0) {
            EXPECT(tok == rt && std::memcmp(lg.data(), rl.data(), (size_t)V * 4) == 0,
                   "slot %d: prefill differs from the batch-1 model (token %d vs %d)", s, tok, rt);
        } else {
            compare(lg.data(), rl, tok, rt, "cached-prefix prefill");
        }
        last[s] = rt;   // both sides continue from the batch-1 model's token
    }
    EXPECT(cache.page_refs(cache.host_block_table(0)[0]) == 2, "shared page refs");
    bool threw = false;
    try {
        runner.prefill(cache, 1, prompts[0]);   // length 19 != 35
    } catch (const std::logic_error&) {
        threw = true;
    }
    EXPECT(threw, "prefill with a length other than the slot's accepted");
    // num_cached beyond the tokens the slot took over by share_prefix: those
    // positions would be read from pages nothing wrote
    EXPECT(cache.cached_tokens(2) == 32 && cache.cached_tokens(1) == 0, "cached token counts");
    threw = false;
    try {
        runner.prefill(cache, 1, prompts[1], nullptr, nullptr, 16);   // slot 1 shares nothing
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    EXPECT(threw, "num_cached beyond the shared prefix accepted");
    threw = false;
    try {
        runner.prefill(cache, 2, prompts[2], nullptr, nullptr, 33);   // 32 shared tokens
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    EXPECT(threw, "num_cached 33 over a 32-token shared prefix accepted");
    for (int st = 0; st < 4; ++st) {
        std::vector<float> lg;
        const std::vector<int32_t> next = runner.decode_step(cache, 4, last, &lg);
        EXPECT(next[3] == -1, "inactive slot got token %d", next[3]);
        for (int s = 0; s < 3; ++s) {
            std::vector<float> rl(V);
            int32_t rt = -1;
            KVHP_CHECK(kvhp_llama_decode_step(ref[s], last[s], rl.data(), &rt));
            char what[64];
            std::snprintf(what, sizeof what, "step %d slot %d", st, s);
            compare(lg.data() + (size_t)s * V, rl, next[s], rt, what);
            EXPECT(cache.seq_len(s) == (int)prompts[s].size() + st + 1, "%s: length", what);
        }
        for (int s = 0; s < 3; ++s) last[s] = next[s];
    }
    for (auto r : ref) kvhp_llama_destroy(r);
    for (int s = 0; s < 3; ++s) cache.release(s);
    EXPECT(cache.free_page_count() == cache.num_pages(), "pages leaked");
}

void case_forward_gpu_mirror() {
    // prefill_gpu / decode_step_gpu (reference forward_gpu.h:88-113) over a
    // KVCache against the library's own batch-1 model of the same weights:
    // logits bit for bit, the cache bytes equal the model's pages, the
    // lengths as the reference sets them, d_last_logits and profiling forms.
    ModelConfig cfg;   // the reference's defaults, then a small Llama shape
    cfg.model_type = "llama";
    cfg.vocab_size = 1024;
    cfg.hidden_size = 256;
    cfg.intermediate_size = 512;
    cfg.num_hidden_layers = 2;
    cfg.num_attention_heads = 4;
    cfg.num_key_value_heads = 2;
    cfg.head_dim = 64;
    cfg.rms_norm_eps = 1e-5f;
    cfg.rope_theta = 10000.f;
    cfg.tie_word_embeddings = false;
    cfg.max_position_embeddings = 96;
    const int M = 96, V = cfg.vocab_size;
    const uint64_t seed = 41;
    ModelWeightsGPU weights;
    EXPECT(weights.init_synthetic(cfg, seed), "init_synthetic: %s", kvhp_last_error());
    ActivationBuffersGPU buffers;
    buffers.allocate(cfg, M);
    KVCache kv(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim, M);
    const kvhp_llama_config c = cfg.to_c();
    void* ref = nullptr;
    KVHP_CHECK(kvhp_llama_create(&c, seed, M, &ref));

    std::mt19937 rng(404);
    std::vector<int64_t> prompt(37);
    std::vector<int32_t> prompt32(prompt.size());
    for (size_t i = 0; i < prompt.size(); ++i) prompt32[i] = (int32_t)(prompt[i] = rng() % V);
    const std::vector<float> lg = prefill_gpu(prompt, cfg, weights, buffers, kv, nullptr);
    std::vector<float> rl(V);
    int32_t tok = -1;
    KVHP_CHECK(kvhp_llama_prefill(ref, prompt32.data(), (int)prompt32.size(), rl.data(), &tok));
    EXPECT(lg.size() == (size_t)V && std::memcmp(lg.data(), rl.data(), (size_t)V * 4) == 0,
           "prefill logits differ");
    EXPECT(kv.current_seq_len() == 37, "length after prefill %d", kv.current_seq_len());
    auto same_cache = [&](const char* what) {
        for (int l = 0; l < cfg.num_hidden_layers; ++l)
            for (int is_v = 0; is_v < 2; ++is_v) {
                void* pool = nullptr;
                size_t n = 0;
                KVHP_CHECK(kvhp_llama_tensor(ref, l, is_v ? KVHP_LLAMA_POOL_V : KVHP_LLAMA_POOL_K,
                                             &pool, &n));
                const size_t per = (size_t)cfg.num_key_value_heads * M * cfg.head_dim;
                EXPECT(n == per, "%s: pool size", what);
                std::vector<half> a(per), b(per);
                HIP_CHECK(hipMemcpy(a.data(), kv.get_layer_ptr(l, is_v), per * 2, hipMemcpyDeviceToHost));
                HIP_CHECK(hipMemcpy(b.data(), pool, per * 2, hipMemcpyDeviceToHost));
                EXPECT(std::memcmp(a.data(), b.data(), per * 2) == 0, "%s: layer %d %c differs",
                       what, l, is_v ? 'V' : 'K');
            }
    };
    same_cache("after prefill");
    int pos = 37;
    for (int st = 0; st < 6; ++st, ++pos) {
        const std::vector<float> dl = decode_step_gpu(tok, pos, cfg, weights, buffers, kv, nullptr);
        int32_t next = -1;
        KVHP_CHECK(kvhp_llama_decode_step(ref, tok, rl.data(), &next));
        EXPECT(std::memcmp(dl.data(), rl.data(), (size_t)V * 4) == 0, "decode step %d logits", st);
        EXPECT(kv.current_seq_len() == pos + 1, "length after step %d", st);
        tok = next;
    }
    same_cache("after decode");
    // device logits: nothing returned, the buffer holds the same values
    DeviceBuffer<float> dlog(V);
    const std::vector<float> none = decode_step_gpu(tok, pos, cfg, weights, buffers, kv, nullptr,
                                                    dlog.data());
    int32_t next = -1;
    KVHP_CHECK(kvhp_llama_decode_step(ref, tok, rl.data(), &next));
    EXPECT(none.empty(), "d_last_logits: host logits returned");
    const std::vector<float> got = download(dlog);
    EXPECT(std::memcmp(got.data(), rl.data(), (size_t)V * 4) == 0, "d_last_logits values");
    std::vector<KernelRecord> rec;
    (void)decode_step_gpu(next, pos + 1, cfg, weights, buffers, kv, nullptr, nullptr, &rec);
    EXPECT(rec.size() == 1 && rec[0].ms > 0.f, "profile records");
    kvhp_llama_destroy(ref);

    // the reference's errors: a prompt longer than the buffers, and this
    // build's: a cache whose max_seq is not whole pages, a wrong shape
    auto throws = [](const std::function<void()>& f) {
        try {
            f();
        } catch (const std::exception&) {
            return true;
        }
        return false;
    };
    ActivationBuffersGPU small;
    small.allocate(cfg, 16);
    EXPECT(throws([&] { prefill_gpu(prompt, cfg, weights, small, kv, nullptr); }),
           "prompt longer than the buffers accepted");
    KVCache odd(cfg.num_hidden_layers, cfg.num_key_value_heads, cfg.head_dim, 90);
    EXPECT(throws([&] { prefill_gpu(prompt, cfg, weights, buffers, odd, nullptr); }),
           "cache of 90 positions accepted");
    KVCache shallow(1, cfg.num_key_value_heads, cfg.head_dim, M);
    EXPECT(throws([&] { decode_step_gpu(1, 0, cfg, weights, buffers, shallow, nullptr); }),
           "cache with the wrong layer count accepted");
    EXPECT(throws([&] { decode_step_gpu(V, 0, cfg, weights, buffers, kv, nullptr); }),
           "token id past the vocabulary accepted");

    // tied embeddings: the LM head is the embedding
    ModelConfig tied = cfg;
    tied.tie_word_embeddings = true;
    ModelWeightsGPU tw;
    EXPECT(tw.init_synthetic(tied, seed, 32), "tied init");
    void *e = nullptr, *h = nullptr;
    size_t ne = 0, nh = 0;
    KVHP_CHECK(kvhp_llama_tensor(tw.handle(), -1, KVHP_LLAMA_EMBED, &e, &ne));
    KVHP_CHECK(kvhp_llama_tensor(tw.handle(), -1, KVHP_LLAMA_LM_HEAD, &h, &nh));
    std::vector<half> he(ne), hh(nh);
    HIP_CHECK(hipMemcpy(he.data(), e, ne * 2, hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(hh.data(), h, nh * 2, hipMemcpyDeviceToHost));
    EXPECT(ne == nh && std::memcmp(he.data(), hh.data(), ne * 2) == 0, "LM head not tied");
}

struct Case {
    const char* name;
    bool gpu;
    void (*fn)();
};

}  // namespace

int main(int argc, char** argv) {
    const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
    const bool cpu = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
    if (!gpu && !cpu) {
        std::fprintf(stderr, "usage: %s --cpu | --gpu\n", argv[0]);
        return 2;
    }
    const Case cases[] = {
        {"half_conversion", false, case_half_conversion},
        {"host_validation", false, case_host_validation},
        {"kv_view_get_ptr", false, case_kv_view_get_ptr},
        {"kv_cache_layout", true, case_kv_cache_layout},
        {"append_kv_cache", true, case_append_kv_cache},
        {"decode_gqa", true, case_decode_gqa},
        {"decode_gqa_split", true, case_decode_gqa_split},
        {"flash_prefill_gqa", true, case_flash_prefill_gqa},
        {"causal_gqa", true, case_causal_gqa},
        {"paged_identity_equals_kvcache", true, case_paged_identity_equals_kvcache},
        {"paged_serving_steps", true, case_paged_serving_steps},
        {"paged_cache_rejects", true, case_paged_cache_rejects},
        {"paged_prefix_sharing", true, case_paged_prefix_sharing},
        {"llama_runner_paged", true, case_llama_runner_paged},
        {"forward_gpu_mirror", true, case_forward_gpu_mirror},
    };
    for (const Case& c : cases) {
        if (c.gpu && !gpu) continue;
        g_case = c.name;
        const int before = g_failures;
        std::printf("case %s ...\n", c.name);
        std::fflush(stdout);
        try {
            c.fn();
        } catch (const std::exception& e) {
            ++g_failures;
            std::printf("  FAIL [%s] exception: %s\n", c.name, e.what());
        }
        std::printf("case %s: %s\n", c.name, g_failures == before ? "ok" : "FAILED");
        std::fflush(stdout);
    }
    std::printf("%d checks, %d failures\n", g_checks, g_failures);
    return g_failures ? 1 : 0;
}
