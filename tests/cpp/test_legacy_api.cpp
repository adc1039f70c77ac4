// The legacy single-head interfaces over the new cache (paged-attention_amd/cpp:
// CpuAttention, PagedPool, PagedPoolAttention, the host fp16 codec), driven the
// way the reference's tests/test_paged_pool.cpp and tests/test_cpu_attention.cpp
// drive theirs, checked against the CPU oracle (oracle/pa_oracle.h).
//
//   test_legacy_api cpu   host-only: fp16 codec against the oracle's (every
//                         half, ties, specials), CpuAttention against the
//                         oracle's cpu_attention and closed forms, the pool's
//                         free sizing helpers
//   test_legacy_api gpu   PagedPool (decode, decode_device) / PagedPoolAttention
//                         on the device
//
// Exit status 0 = every check passed; each failure prints one line.

#include "cpu_attention.hpp"
#include "decode/half_host.hpp"
#include "pa_oracle.h"
#include "paged_pool.hpp"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

int g_failures = 0;

void expect(bool ok, const std::string& what) {
    if (!ok) {
        std::printf("FAIL: %s\n", what.c_str());
        ++g_failures;
    }
}

template <class E, class F>
void expect_throw(F&& f, const std::string& what) {
    try {
        f();
        expect(false, what + " (no exception)");
    } catch (const E&) {
    } catch (const std::exception& e) {
        expect(false, what + " (wrong exception: " + e.what() + ")");
    }
}

uint32_t bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, sizeof u);
    return u;
}
float from_bits(uint32_t u) {
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
}

struct Inputs {
    std::vector<float> q, K, V;
};

// N(0,1) q, K, V for one head ([d], [T][d], [T][d]).
Inputs make_inputs(int d, int T, uint32_t seed) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> nd(0.f, 1.f);
    Inputs in;
    in.q.resize(static_cast<size_t>(d));
    in.K.resize(static_cast<size_t>(T) * d);
    in.V.resize(static_cast<size_t>(T) * d);
    for (auto& x : in.q) x = nd(rng);
    for (auto& x : in.K) x = nd(rng);
    for (auto& x : in.V) x = nd(rng);
    return in;
}

std::vector<float> round_f16(const std::vector<float>& x) {
    std::vector<float> r(x.size());
    for (size_t i = 0; i < x.size(); ++i) r[i] = orc_f16_to_f32(orc_f32_to_f16(x[i]));
    return r;
}

double max_abs(const std::vector<float>& a, const std::vector<float>& b) {
    double m = 0;
    for (size_t i = 0; i < a.size(); ++i) m = std::max(m, std::fabs(double(a[i]) - double(b[i])));
    return m;
}

// ---- host-only checks ------------------------------------------------------

void cpu_checks() {
    // Every half decodes like the oracle's decoder (NaN payloads by bits).
    for (uint32_t h = 0; h < 65536; ++h) {
        const float a = decode::f16_to_f32(static_cast<uint16_t>(h));
        const float b = orc_f16_to_f32(static_cast<uint16_t>(h));
        if (bits(a) != bits(b) && !(std::isnan(a) && std::isnan(b))) {
            expect(false, "f16_to_f32 differs at " + std::to_string(h));
            break;
        }
    }
    // Encode: every half value, the midpoints between neighbours (ties), one
    // float ulp either side of them, specials, and random floats of all exponents.
    std::vector<float> xs;
    for (uint32_t h = 0; h < 0x7c00u; ++h) {
        const float v  = orc_f16_to_f32(static_cast<uint16_t>(h));
        const float nx = orc_f16_to_f32(static_cast<uint16_t>(h + 1));
        const float mid = h + 1 < 0x7c00u ? (v + nx) / 2 : 65520.0f;
        for (float x : {v, mid, from_bits(bits(mid) + 1), from_bits(bits(mid) - 1)}) {
            xs.push_back(x);
            xs.push_back(-x);
        }
    }
    for (float x : {INFINITY, -INFINITY, NAN, 65519.99f, 65520.0f, 1e30f, 1e-30f, 0.0f, -0.0f,
                    std::ldexp(1.0f, -25), std::ldexp(1.0f, -26), std::ldexp(1.5f, -25), std::ldexp(1.0f, -14)})
        xs.push_back(x);
    std::mt19937 rng(7);
    for (int i = 0; i < 1000000; ++i) xs.push_back(from_bits(rng()));
    int bad = 0;
    for (float x : xs) {
        const uint16_t a = decode::f32_to_f16(x), b = orc_f32_to_f16(x);
        const bool both_nan = std::isnan(x) && (a & 0x7c00u) == 0x7c00u && (a & 0x3ffu) && (b & 0x7c00u) == 0x7c00u &&
                              (b & 0x3ffu);
        if (a != b && !both_nan && bad++ < 5) expect(false, "f32_to_f16 differs at " + std::to_string(x));
    }
    expect(bad == 0, std::to_string(bad) + " f32_to_f16 mismatches");

    // CpuAttention = the oracle's cpu_attention (same operation order, so bitwise).
    CpuAttention cpu;
    expect(std::string(cpu.name()) == "cpu", "CpuAttention name");
    for (uint32_t seed : {1u, 2u, 3u})
        for (int d : {8, 64, 128})
            for (int T : {1, 4, 32, 256, 1024}) {
                const Inputs in = make_inputs(d, T, seed);
                std::vector<float> a(static_cast<size_t>(d)), b(static_cast<size_t>(d));
                cpu.run(in.q.data(), in.K.data(), in.V.data(), a.data(), T, d);
                orc_cpu_attention(in.q.data(), in.K.data(), in.V.data(), b.data(), T, d);
                expect(std::memcmp(a.data(), b.data(), sizeof(float) * a.size()) == 0,
                       "CpuAttention == oracle (d " + std::to_string(d) + ", T " + std::to_string(T) + ")");
            }
    // Closed forms (tests/test_cpu_attention.cpp): one token returns its V row;
    // identical keys average V.
    {
        const Inputs in = make_inputs(16, 1, 9);
        std::vector<float> o(16);
        cpu.run(in.q.data(), in.K.data(), in.V.data(), o.data(), 1, 16);
        expect(o == in.V, "T = 1 returns V");
        Inputs u = make_inputs(16, 5, 10);
        for (int t = 1; t < 5; ++t) std::copy(u.K.begin(), u.K.begin() + 16, u.K.begin() + t * 16);
        cpu.run(u.q.data(), u.K.data(), u.V.data(), o.data(), 5, 16);
        for (int i = 0; i < 16; ++i) {
            float m = 0;
            for (int t = 0; t < 5; ++t) m += u.V[static_cast<size_t>(t) * 16 + i];
            expect(std::fabs(o[static_cast<size_t>(i)] - m / 5) < 1e-6f, "identical keys average V");
        }
    }
}

// ---- device checks -----------------------------------------------------------

constexpr int kD = 128;

// pool.hpp:63-72's free helpers: closed forms for this pool's element sizes.
void helper_checks() {
    expect(paged_waste_tokens(17) == 15 && paged_waste_tokens(16) == 0 && paged_waste_tokens(1) == 15 &&
               paged_waste_tokens(5, 4) == 3 && paged_waste_tokens(8192, 8192) == 0,
           "paged_waste_tokens closed forms");
    const size_t gib = size_t{1} << 30;
    // 1 GiB of fp16 pages of 16 x 128: 2 * 2 * 16 * 128 = 8 KiB per page, 131072
    // pages; 1024 tokens = 64 pages per sequence.
    expect(paged_max_sequences_for_budget(gib, 1024, 128) == 2048, "budget helper, fp16");
    expect(paged_max_sequences_for_budget(gib, 1024, 128, 16, decode::KVDtype::FP8_E4M3) == 4096,
           "budget helper, FP8 (one byte per element)");
    expect(paged_max_sequences_for_budget(gib, 1025, 128) == 131072 / 65, "budget helper rounds pages up");
    expect(paged_max_sequences_for_budget(1000, 16, 128) == 0, "a budget below one page holds no sequence");
    expect_throw<std::invalid_argument>([] { paged_max_sequences_for_budget(1 << 20, 0, 128); },
                                        "budget helper rejects a zero length");
}

void gpu_checks() {
    CpuAttention       cpu;
    PagedPoolAttention paged;
    expect(std::string(paged.name()) == "paged_pool", "PagedPoolAttention name");
    // MatchesCpuReference (test_paged_pool.cpp): d = 128 only; fp16 storage,
    // so 2e-3 against fp32 attention over the given rows and 1e-3 against
    // fp32 attention over the rows rounded to fp16.
    for (uint32_t seed : {1u, 2u, 3u})
        for (int T : {1, 4, 15, 16, 17, 32, 256, 1024, 4099}) {
            const Inputs in = make_inputs(kD, T, seed);
            std::vector<float> got(kD), ref(kD), ref16(kD);
            paged.run(in.q.data(), in.K.data(), in.V.data(), got.data(), T, kD);
            cpu.run(in.q.data(), in.K.data(), in.V.data(), ref.data(), T, kD);
            const auto q16 = round_f16(in.q), K16 = round_f16(in.K), V16 = round_f16(in.V);
            cpu.run(q16.data(), K16.data(), V16.data(), ref16.data(), T, kD);
            char buf[128];
            std::snprintf(buf, sizeof buf, "paged vs cpu (T %d, seed %u): %.3g / %.3g", T, seed, max_abs(got, ref),
                          max_abs(got, ref16));
            expect(max_abs(got, ref) < 2e-3 && max_abs(got, ref16) < 1e-3, buf);
        }
    expect_throw<std::invalid_argument>([] { PagedPool p(4, 1, 4, 64); }, "head_dim 64 is rejected");

    // AdmitAndRelease / PoolFullWhenNoPagesLeft / PagesRecycledAfterRelease.
    {
        const int T = 32, pages = (T + PAGE_SIZE - 1) / PAGE_SIZE;
        PagedPool pool(pages * 4, 4, pages * 2, kD);
        std::vector<float> K(static_cast<size_t>(T) * kD, 0.f), V(K);
        const int s0 = pool.admit(K.data(), V.data(), T), s1 = pool.admit(K.data(), V.data(), T);
        expect(s0 >= 0 && s1 >= 0 && s0 != s1, "two admits");
        expect(pool.is_occupied(s0) && pool.actual_len(s0) == T, "occupied with its length");
        const int free_before = pool.free_page_count();
        pool.release(s0);
        expect(!pool.is_occupied(s0) && pool.free_page_count() > free_before, "release frees pages");
        expect(pool.admit(K.data(), V.data(), T) >= 0, "admit after release");
        expect(pool.total_pages() == pages * 4 && pool.max_sequences() == 4 && pool.d() == kD, "accessors");
        expect(pool.total_kv_bytes() == 2ull * pages * 4 * PAGE_SIZE * kD * 2, "total_kv_bytes (fp16)");
        expect_throw<std::invalid_argument>([&] { pool.admit(K.data(), V.data(), 0); }, "admit of 0 rows");
        expect_throw<std::invalid_argument>([&] { pool.release(3); }, "release of a free slot");
    }
    {
        std::vector<float> K(static_cast<size_t>(PAGE_SIZE) * kD, 0.f), V(K);
        PagedPool pool(2, 4, 4, kD);
        expect(pool.admit(K.data(), V.data(), PAGE_SIZE) >= 0 && pool.admit(K.data(), V.data(), PAGE_SIZE) >= 0,
               "two one-page admits");
        expect(pool.admit(K.data(), V.data(), PAGE_SIZE) == -1, "third admit finds no page");
        expect(!pool.is_occupied(2), "a refused admit leaves its slot free");
        PagedPool one(1, 2, 2, kD);
        const int s = one.admit(K.data(), V.data(), PAGE_SIZE);
        expect(s >= 0 && one.free_page_count() == 0, "one page taken");
        one.release(s);
        expect(one.free_page_count() == 1 && one.admit(K.data(), V.data(), PAGE_SIZE) >= 0, "page recycled");
    }
    // MultipleSlots_IndependentResults and AppendToken.
    {
        const int T = 64, pages = (T + PAGE_SIZE - 1) / PAGE_SIZE;
        PagedPool pool(pages * 4, 4, pages * 2, kD);
        const Inputs a = make_inputs(kD, T, 1), b = make_inputs(kD, T, 2);
        const int s0 = pool.admit(a.K.data(), a.V.data(), T), s1 = pool.admit(b.K.data(), b.V.data(), T);
        std::vector<float> o0(kD), o1(kD);
        pool.decode(s0, a.q.data(), o0.data());
        pool.decode(s1, a.q.data(), o1.data());
        expect(max_abs(o0, o1) > 1e-6, "slots hold their own rows");
    }
    {
        const int T = 2 * PAGE_SIZE;
        PagedPool pool(4, 2, 8, kD);
        const Inputs in = make_inputs(kD, T, 42);
        const int slot = pool.admit(in.K.data(), in.V.data(), T - 1);
        pool.append_token(slot, T - 1, in.K.data() + static_cast<size_t>(T - 1) * kD,
                          in.V.data() + static_cast<size_t>(T - 1) * kD);
        expect(pool.actual_len(slot) == T, "append_token grows the slot");
        std::vector<float> got(kD), whole(kD), ref(kD);
        pool.decode(slot, in.q.data(), got.data());
        PagedPoolAttention().run(in.q.data(), in.K.data(), in.V.data(), whole.data(), T, kD);
        CpuAttention().run(in.q.data(), in.K.data(), in.V.data(), ref.data(), T, kD);
        expect(got == whole, "admit + append_token == admitting every row (bitwise)");
        expect(max_abs(got, ref) < 2e-3, "append_token vs cpu");
        expect_throw<std::invalid_argument>(
            [&] { pool.append_token(slot, T - 1, in.K.data(), in.V.data()); }, "append_token at a stale position");
        // Fill the remaining pages token by token, then one more has no page.
        for (int t = T; t < 4 * PAGE_SIZE; ++t) pool.append_token(slot, t, in.K.data(), in.V.data());
        expect(pool.free_page_count() == 0, "pool full");
        expect_throw<std::length_error>(
            [&] { pool.append_token(slot, 4 * PAGE_SIZE, in.K.data(), in.V.data()); }, "append_token without a page");
        expect(pool.actual_len(slot) == 4 * PAGE_SIZE, "a refused append_token changes nothing");
    }
    // decode_device (pool.hpp:21-24): fp32 device q / out, the first actual_len
    // rows of a slot, no synchronization. Whole length: bitwise equal to
    // decode(); a prefix: bitwise equal to a pool holding only the prefix.
    {
        const int T = 300, Tp = 129;
        PagedPool pool(64, 3, 32, kD);
        const Inputs in = make_inputs(kD, T, 77), other = make_inputs(kD, T, 78);
        const int s_other = pool.admit(other.K.data(), other.V.data(), T);
        const int slot = pool.admit(in.K.data(), in.V.data(), T);
        expect(s_other >= 0 && slot >= 0 && slot != s_other, "two slots for decode_device");
        float *dq = nullptr, *dout = nullptr;
        HIP_CHECK(hipMalloc(&dq, sizeof(float) * kD));
        HIP_CHECK(hipMalloc(&dout, sizeof(float) * 2 * kD));
        HIP_CHECK(hipMemcpy(dq, in.q.data(), sizeof(float) * kD, hipMemcpyHostToDevice));
        pool.decode_device(slot, T, dq, dout);
        pool.decode_device(slot, Tp, dq, dout + kD, nullptr, nullptr, nullptr);
        HIP_CHECK(hipDeviceSynchronize());
        std::vector<float> whole(kD), prefix(kD), host(kD), ref_prefix(kD), ref(kD);
        HIP_CHECK(hipMemcpy(whole.data(), dout, sizeof(float) * kD, hipMemcpyDeviceToHost));
        HIP_CHECK(hipMemcpy(prefix.data(), dout + kD, sizeof(float) * kD, hipMemcpyDeviceToHost));
        pool.decode(slot, in.q.data(), host.data());
        expect(whole == host, "decode_device over the whole slot == decode (bitwise)");
        PagedPool small(16, 1, 16, kD);
        const int sp = small.admit(in.K.data(), in.V.data(), Tp);
        small.decode(sp, in.q.data(), ref_prefix.data());
        expect(prefix == ref_prefix, "decode_device over a prefix == a pool of the prefix (bitwise)");
        const auto q16 = round_f16(in.q), K16 = round_f16(in.K), V16 = round_f16(in.V);
        CpuAttention().run(q16.data(), K16.data(), V16.data(), ref.data(), Tp, kD);
        expect(max_abs(prefix, ref) < 2e-3, "decode_device prefix vs cpu");
        expect_throw<std::invalid_argument>([&] { pool.decode_device(slot, T + 1, dq, dout); },
                                            "decode_device past the slot's length");
        expect_throw<std::invalid_argument>([&] { pool.decode_device(slot, 0, dq, dout); }, "decode_device of 0 rows");
        expect_throw<std::invalid_argument>([&] { pool.decode_device(2, 1, dq, dout); }, "decode_device of a free slot");
        // The device pools: distinct, V laid out after K.
        const auto* kb = static_cast<const unsigned char*>(pool.kv_K_base());
        const auto* vb = static_cast<const unsigned char*>(pool.kv_V_base());
        expect(kb && vb && vb >= kb + pool.total_kv_bytes() / 2, "kv_K_base / kv_V_base");
        HIP_CHECK(hipFree(dq));
        HIP_CHECK(hipFree(dout));
    }
    // An FP8 pool: E4M3 of the fp16-rounded rows times 1/scale; compared with
    // fp32 attention over the same quantized values.
    {
        const int T = 300;
        const float scale = 4.0f / 448.0f, inv = 1.0f / scale;
        PagedPool pool(32, 1, 32, kD, PAGE_SIZE, decode::KVDtype::FP8_E4M3, scale, scale);
        const Inputs in = make_inputs(kD, T, 5);
        const int slot = pool.admit(in.K.data(), in.V.data(), T);
        std::vector<float> got(kD), ref(kD), Kq(in.K.size()), Vq(in.V.size());
        for (size_t i = 0; i < Kq.size(); ++i) {
            Kq[i] = orc_e4m3_to_f32(orc_f32_to_e4m3(orc_f16_to_f32(orc_f32_to_f16(in.K[i])) * inv)) * scale;
            Vq[i] = orc_e4m3_to_f32(orc_f32_to_e4m3(orc_f16_to_f32(orc_f32_to_f16(in.V[i])) * inv)) * scale;
        }
        pool.decode(slot, in.q.data(), got.data());
        const auto q16 = round_f16(in.q);
        CpuAttention().run(q16.data(), Kq.data(), Vq.data(), ref.data(), T, kD);
        expect(max_abs(got, ref) < 2e-3, "FP8 pool vs cpu over the quantized rows");
    }
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    try {
        cpu_checks();
        helper_checks();
        if (mode == "gpu") gpu_checks();
    } catch (const std::exception& e) {
        std::printf("FAIL: unexpected exception: %s\n", e.what());
        ++g_failures;
    }
    std::printf("%s: %d failure(s)\n", mode.c_str(), g_failures);
    return g_failures == 0 ? 0 : 1;
}
