// Drives the C++ surface (paged-attention_amd/cpp: decode::PagedKVCache,
// make_plan, DevicePlan, paged_decode, the reference's exception types) the way
// the reference's tests/test_paged_decode.cu does, and checks results against
// the CPU oracle (oracle/pa_oracle.h).
//
//   test_cpp_api cpu   host-only checks (planner, validation, error mapping)
//   test_cpp_api gpu   decode on the device through PagedKVCache and through
//                      DecodeParams + DevicePlan + paged_decode
//
// Exit status 0 = every check passed; each failure prints one line.

#include "decode/paged_kv_cache.hpp"
#include "kv_store.hpp"
#include "pa_oracle.h"

#include <hip/hip_runtime.h>

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

constexpr int kD = 128;

// ---- host-only checks ------------------------------------------------------

void cpu_checks() {
    using namespace decode;
    // decode.hpp:29-39 on the host: explicit grids need no device.
    const std::vector<int> lens = {5000, 90, 1, 700};
    const int tile = tile_tokens(KVDtype::FP16, kD, 4);
    expect(tile == 16 || tile == 32, "tile_tokens is the kernel step");
    DecodePlan p = make_plan(KVDtype::FP16, lens, 32, 8, kD, 7);
    expect(p.num_ctas <= 7 && p.num_ctas > 0, "make_plan honours the requested grid");
    expect(p.cta_seg_begin.size() == static_cast<size_t>(p.num_ctas) + 1, "cta prefix size");
    expect(p.item_seg_begin.size() == lens.size() * 8 + 1, "item prefix size");
    expect(p.item_seg_begin.back() == static_cast<int>(p.segments.size()), "item prefix ends at segments");
    // Segments partition every (row, head) in token order.
    for (size_t b = 0; b < lens.size(); ++b)
        for (int h = 0; h < 8; ++h) {
            const int i = static_cast<int>(b) * 8 + h;
            int at = 0;
            for (int s = p.item_seg_begin[i]; s < p.item_seg_begin[i + 1]; ++s) {
                const int4 sg = p.segments[static_cast<size_t>(s)];
                expect(sg.x == static_cast<int>(b) && sg.y == h && sg.z == at && sg.w > sg.z, "segment order");
                at = sg.w;
            }
            expect(at == lens[b], "segments cover the row");
        }
    // The reference's error types (decode.cu:30-36, :68, :79).
    expect_throw<std::invalid_argument>([] { make_plan(KVDtype::FP16, {16}, 32, 8, 64, 4); }, "head_dim 64");
    expect_throw<std::invalid_argument>([] { make_plan(KVDtype::FP16, {16}, 24, 8, kD, 4); }, "group 3");
    expect_throw<std::invalid_argument>([] { make_plan(KVDtype::FP16, {16}, 30, 8, kD, 4); }, "hq % hkv");
    expect_throw<std::invalid_argument>([] { make_plan(KVDtype::FP16, {16, 0}, 32, 8, kD, 4); }, "empty sequence");
    // DecodeParams matches the ABI struct field for field.
    DecodeParams dp{};
    dp.page_size = 16;
    dp.v_scale   = 0.5f;
    expect(detail::abi(dp)->page_size == 16 && detail::abi(dp)->v_scale == 0.5f, "DecodeParams layout");
}

// ---- device checks -----------------------------------------------------------

std::vector<uint16_t> normal_f16(std::mt19937& rng, size_t n) {
    std::normal_distribution<float> nd(0.f, 1.f);
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = orc_f32_to_f16(nd(rng));
    return v;
}

template <class T>
T* to_device(const std::vector<T>& h) {
    T* d = nullptr;
    HIP_CHECK(hipMalloc(&d, sizeof(T) * (h.empty() ? 1 : h.size())));
    if (!h.empty()) HIP_CHECK(hipMemcpy(d, h.data(), sizeof(T) * h.size(), hipMemcpyHostToDevice));
    return d;
}

template <class T>
std::vector<T> to_host(const T* d, size_t n) {
    std::vector<T> h(n);
    HIP_CHECK(hipMemcpy(h.data(), d, sizeof(T) * n, hipMemcpyDeviceToHost));
    return h;
}

// tests/test_paged_decode.cu:50-151 run_case through decode::PagedKVCache:
// append (whole or round-robin chunks; with `batched` every round of chunks is
// one append_batch call), decode, then compare with the oracle over the stored
// cache contents. Returns the max-abs error.
double run_case(decode::KVDtype dtype, int hq, int hkv, int page, const std::vector<int>& lens, int chunk,
                int ctas, bool shuffle, bool batched) {
    using namespace decode;
    std::mt19937 rng(1234);
    const int B = static_cast<int>(lens.size());
    std::vector<std::vector<uint16_t>> K, V;
    int pages = 0, max_pages = 0;
    for (int L : lens) {
        K.push_back(normal_f16(rng, static_cast<size_t>(L) * hkv * kD));
        V.push_back(normal_f16(rng, static_cast<size_t>(L) * hkv * kD));
        pages += (L + page - 1) / page;
        max_pages = std::max(max_pages, (L + page - 1) / page);
    }
    const std::vector<uint16_t> q = normal_f16(rng, static_cast<size_t>(B) * hq * kD);
    PagedKVCache::Config cfg{};
    cfg.num_pages          = pages + 3;
    cfg.page_size          = page;
    cfg.num_kv_heads       = hkv;
    cfg.head_dim           = kD;
    cfg.max_slots          = B;
    cfg.max_pages_per_slot = max_pages;
    cfg.dtype              = dtype;
    cfg.k_scale = cfg.v_scale = 4.0f / 448.0f;
    PagedKVCache cache(cfg);
    if (shuffle) cache.shuffle_free_pages(7);
    std::vector<uint16_t*> dK, dV;
    for (int b = 0; b < B; ++b) {
        expect(cache.admit() == b, "admit order");
        dK.push_back(to_device(K[static_cast<size_t>(b)]));
        dV.push_back(to_device(V[static_cast<size_t>(b)]));
    }
    std::vector<int> done(static_cast<size_t>(B), 0);
    const size_t row = static_cast<size_t>(hkv) * kD;
    uint16_t *bk = nullptr, *bv = nullptr;   // one round's tokens, concatenated
    size_t total = 0;
    for (int L : lens) total += static_cast<size_t>(L);
    if (batched) {
        HIP_CHECK(hipMalloc(&bk, sizeof(uint16_t) * total * row));
        HIP_CHECK(hipMalloc(&bv, sizeof(uint16_t) * total * row));
    }
    for (bool more = true; more;) {
        more = false;
        std::vector<int> slots, counts;
        size_t at = 0;
        for (int b = 0; b < B; ++b) {
            const int n = std::min(chunk > 0 ? chunk : lens[b], lens[b] - done[b]);
            if (n <= 0) continue;
            const size_t off = static_cast<size_t>(done[b]) * row;
            if (batched) {
                HIP_CHECK(hipMemcpy(bk + at * row, dK[b] + off, sizeof(uint16_t) * n * row, hipMemcpyDeviceToDevice));
                HIP_CHECK(hipMemcpy(bv + at * row, dV[b] + off, sizeof(uint16_t) * n * row, hipMemcpyDeviceToDevice));
                slots.push_back(b);
                counts.push_back(n);
                at += static_cast<size_t>(n);
            } else {
                expect(cache.append(b, reinterpret_cast<const half*>(dK[b] + off),
                                    reinterpret_cast<const half*>(dV[b] + off), n),
                       "append fits");
            }
            done[b] += n;
            more = true;
        }
        if (!slots.empty())
            expect(cache.append_batch(slots, counts, reinterpret_cast<const half*>(bk),
                                      reinterpret_cast<const half*>(bv)),
                   "append_batch fits");
        // The next round's copies overwrite bk / bv (null stream, which waits for the batch kernel).
    }
    for (int b = 0; b < B; ++b) expect(cache.seq_len(b) == lens[b], "seq_len after append");
    uint16_t* dq = to_device(q);
    uint16_t* dout = nullptr;
    HIP_CHECK(hipMalloc(&dout, sizeof(uint16_t) * q.size()));
    cache.decode(reinterpret_cast<const half*>(dq), reinterpret_cast<half*>(dout), B, hq, ctas);
    HIP_CHECK(hipDeviceSynchronize());
    const std::vector<uint16_t> out = to_host(dout, q.size());
    expect(ctas == 0 || cache.last_plan().num_ctas <= ctas, "plan respects the grid");

    // Oracle over the stored bytes.
    const DecodeParams p = cache.params();
    const size_t pool = static_cast<size_t>(cfg.num_pages) * hkv * page * kD * kv_dtype_bytes(dtype);
    const std::vector<uint8_t> kc = to_host(static_cast<const uint8_t*>(p.k_cache), pool);
    const std::vector<uint8_t> vc = to_host(static_cast<const uint8_t*>(p.v_cache), pool);
    std::vector<int32_t> table(static_cast<size_t>(B) * max_pages, 0);
    for (int b = 0; b < B; ++b) {
        const std::vector<int>& t = cache.block_table(b);
        std::copy(t.begin(), t.end(), table.begin() + static_cast<long>(b) * max_pages);
    }
    std::vector<float> ref(q.size());
    orc_paged_decode(static_cast<int>(dtype), q.data(), kc.data(), vc.data(), table.data(), max_pages, nullptr,
                     lens.data(), B, hq, hkv, kD, page, cfg.k_scale, cfg.v_scale, ref.data(), 8);
    double err = 0;
    for (size_t i = 0; i < out.size(); ++i) err = std::max(err, std::fabs(double(orc_f16_to_f32(out[i])) - ref[i]));

    // The same step through DecodeParams + make_plan + DevicePlan + paged_decode.
    DecodeParams dp = cache.params();
    std::vector<int32_t> slots(static_cast<size_t>(B));
    for (int b = 0; b < B; ++b) slots[static_cast<size_t>(b)] = b;
    DecodePlan plan = make_plan(dtype, lens, hq, hkv, kD, ctas);
    DevicePlan dplan;
    dplan.upload(plan, hq / hkv, kD);
    dplan.bind(dp);
    uint16_t* dout2 = nullptr;
    HIP_CHECK(hipMalloc(&dout2, sizeof(uint16_t) * q.size()));
    dp.q           = reinterpret_cast<const half*>(dq);
    dp.out         = reinterpret_cast<half*>(dout2);
    dp.slot_ids    = nullptr;
    dp.batch       = B;
    dp.num_q_heads = hq;
    paged_decode(dtype, dp);
    HIP_CHECK(hipDeviceSynchronize());
    const std::vector<uint16_t> out2 = to_host(dout2, q.size());
    expect(std::memcmp(out.data(), out2.data(), out.size() * 2) == 0, "PagedKVCache::run == paged_decode");

    for (int b = 0; b < B; ++b) {
        HIP_CHECK(hipFree(dK[b]));
        HIP_CHECK(hipFree(dV[b]));
    }
    HIP_CHECK(hipFree(dq));
    HIP_CHECK(hipFree(dout));
    HIP_CHECK(hipFree(dout2));
    if (bk) HIP_CHECK(hipFree(bk));
    if (bv) HIP_CHECK(hipFree(bv));
    return err;
}

void gpu_checks() {
    using decode::KVDtype;
    struct Case {
        KVDtype dt;
        int hq, hkv, page;
        std::vector<int> lens;
        int chunk, ctas;
        bool shuffle;
        bool batched = false;
    };
    const std::vector<Case> cases = {
        {KVDtype::FP16, 32, 8, 16, {1}, 0, 0, false},
        {KVDtype::FP8_E4M3, 32, 8, 16, {1}, 0, 0, false},
        {KVDtype::FP16, 8, 1, 16, {777}, 0, 0, false},
        {KVDtype::FP16, 32, 8, 16, {1, 15, 16, 17, 129, 1000, 4099}, 0, 0, false},
        {KVDtype::FP8_E4M3, 32, 8, 16, {1, 15, 16, 17, 129, 1000, 4099}, 0, 0, false},
        {KVDtype::FP16, 16, 4, 8, {300, 2500}, 0, 0, false},
        {KVDtype::FP16, 16, 4, 128, {300, 2500}, 0, 0, false},
        {KVDtype::FP8_E4M3, 32, 8, 16, {5000, 90, 1, 700}, 0, 7, false},
        {KVDtype::FP16, 32, 8, 16, {400, 333, 612}, 5, 0, true},
        {KVDtype::FP8_E4M3, 32, 8, 16, {400, 333, 612}, 1, 0, true, true},
        {KVDtype::FP16, 16, 4, 8, {40, 1, 95}, 3, 0, true, true},
    };
    for (size_t i = 0; i < cases.size(); ++i) {
        const Case& c = cases[i];
        const double err = run_case(c.dt, c.hq, c.hkv, c.page, c.lens, c.chunk, c.ctas, c.shuffle, c.batched);
        char buf[160];
        std::snprintf(buf, sizeof buf, "case %zu (%s, hq %d hkv %d page %d): max|gpu - oracle| = %.3g", i,
                      decode::kv_dtype_name(c.dt), c.hq, c.hkv, c.page, err);
        std::printf("%s\n", buf);
        expect(err < 2e-3, buf);
    }

    // tests/test_paged_decode.cu:206-221: a 2-page pool takes 32 tokens, the
    // 33rd append is refused and changes nothing; release returns both pages.
    decode::PagedKVCache::Config cfg{};
    cfg.num_pages = 2;
    cfg.page_size = 16;
    cfg.num_kv_heads = 8;
    cfg.head_dim = kD;
    cfg.max_slots = 2;
    cfg.max_pages_per_slot = 4;
    decode::PagedKVCache cache(cfg);
    std::vector<uint16_t> kv(static_cast<size_t>(33) * 8 * kD, 0x3c00);
    uint16_t* d = to_device(kv);
    const int slot = cache.admit();
    expect(cache.append(slot, reinterpret_cast<const half*>(d), reinterpret_cast<const half*>(d), 32), "32 tokens fit");
    expect(!cache.append(slot, reinterpret_cast<const half*>(d), reinterpret_cast<const half*>(d), 1), "33rd refused");
    expect(cache.seq_len(slot) == 32 && cache.free_pages() == 0, "refused append changes nothing");
    cache.release(slot);
    expect(cache.free_pages() == 2 && !cache.occupied(slot), "release returns the pages");
    expect_throw<std::length_error>(
        [&] {
            const int s2 = cache.admit();
            cache.append(s2, reinterpret_cast<const half*>(d), reinterpret_cast<const half*>(d), 65);
        },
        "append past max_pages_per_slot");
    HIP_CHECK(hipFree(d));

    // ContiguousKVStore round trip (include/kv_store.hpp).
    std::vector<float> hk(4 * kD, 1.5f), hv(4 * kD, -2.f);
    ContiguousKVStore store(hk.data(), hv.data(), 4, kD);
    const std::vector<float> back = to_host(store.accessor().V, hv.size());
    expect(back == hv, "ContiguousKVStore copies to the device");
}

}  // namespace

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    try {
        cpu_checks();
        if (mode == "gpu") gpu_checks();
    } catch (const std::exception& e) {
        std::printf("FAIL: unexpected exception: %s\n", e.what());
        ++g_failures;
    }
    std::printf("%s: %d failure(s)\n", mode.c_str(), g_failures);
    return g_failures == 0 ? 0 : 1;
}
