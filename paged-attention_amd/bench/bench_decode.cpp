// Native bench CLI of the paged split-KV decode path on MI355X: the modes,
// flags and CSV columns of the reference's bench/bench_decode.cu:1-16, over the
// C++ surface (decode::PagedKVCache) of libpa_decode.so. CSV on stdout,
// '#' comments on stderr.
//
//   bench_decode sweep     [--dtype fp16|fp8]    batch x seq_len sweep
//   bench_decode ctas      --batch B --len L      persistent-grid sweep
//   bench_decode pagesize  --batch B --len L      page-size sweep
//   bench_decode capacity  [--budget-gib G]      sequences per KV budget
//   bench_decode copy                            attainable read bandwidth
//   bench_decode single    --batch B --len L     one configuration
//
// Common flags: --hq 32 --hkv 8 --dim 128 --page 16 --iters 50 --dtype fp16|fp8
//               --ctas N (0 = default grid) --contiguous-pages --peak-gbps X|device (8000)
//
// Timing (bench_decode.cu:120-139): the step is planned once; each iteration
// streams a 1 GiB buffer first (more than L2 plus the 256 MiB Infinity Cache),
// then times decode + merge with HIP events; the median is reported. Bandwidth
// counts the bytes the step must move (bench_decode.cu:186-191). K/V are
// N(0,1) rounded to fp16, distinct per sequence, generated on the device and
// appended through PagedKVCache::append (FP8: per-tensor amax/448 scales).

#include "decode/paged_kv_cache.hpp"
#include "hip_check.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cerrno>
#include <climits>
#include <cstring>
#include <iterator>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace {

// ---- device data generation -------------------------------------------------

__device__ __forceinline__ uint32_t mix32(uint32_t x) {   // a 32-bit integer hash (xorshift-multiply)
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}

// x[i] = N(0,1) sample (Box-Muller over two hashed uniforms) rounded to fp16.
__global__ void fill_normal_f16(__half* x, size_t n, uint32_t seed) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint32_t a = mix32(static_cast<uint32_t>(i) * 2u + seed * 0x9e3779b9u + static_cast<uint32_t>(i >> 31));
        const uint32_t b = mix32(a ^ 0x68e31da4u);
        const float u1 = (static_cast<float>(a >> 8) + 1.0f) * (1.0f / 16777217.0f);   // (0, 1]
        const float u2 = static_cast<float>(b >> 8) * (1.0f / 16777216.0f);
        x[i] = __float2half(sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2));
    }
}

// *amax = max |x| over n fp16 values (non-negative floats order like their bits).
__global__ void abs_max_f16(const __half* x, size_t n, unsigned int* amax) {
    float m = 0.0f;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        m = fmaxf(m, fabsf(__half2float(x[i])));
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0) atomicMax(amax, __float_as_uint(m));
}

// ---- command line -------------------------------------------------------------
// Every option is a typed field with its default. "--name value" and
// "--name=value" both work; switches take no value. An unknown option, a
// missing or malformed value, or a stray argument is an error: the usage goes
// to stderr and the CLI exits with status 2.

struct Options {
    std::string mode = "sweep";
    int batch = 32, len = 4096, hq = 32, hkv = 8, dim = 128, page = 16, iters = 50, ctas = 0, max_len = 8192;
    double budget_gib = 1.0;
    std::string dtype;           // "" = both dtypes in sweep, fp16 elsewhere
    std::string peak = "8000";   // GB/s, or "device": memory clock x bus width
    bool contiguous_pages = false;
    bool help = false;
};

struct OptionSpec {
    const char* name;
    enum Kind { Int, Real, Text, Switch } kind;
    void* field;
};

std::vector<OptionSpec> option_specs(Options& o) {
    return {{"batch", OptionSpec::Int, &o.batch},          {"len", OptionSpec::Int, &o.len},
            {"hq", OptionSpec::Int, &o.hq},                {"hkv", OptionSpec::Int, &o.hkv},
            {"dim", OptionSpec::Int, &o.dim},              {"page", OptionSpec::Int, &o.page},
            {"iters", OptionSpec::Int, &o.iters},          {"ctas", OptionSpec::Int, &o.ctas},
            {"max-len", OptionSpec::Int, &o.max_len},      {"budget-gib", OptionSpec::Real, &o.budget_gib},
            {"dtype", OptionSpec::Text, &o.dtype},         {"peak-gbps", OptionSpec::Text, &o.peak},
            {"contiguous-pages", OptionSpec::Switch, &o.contiguous_pages},
            {"help", OptionSpec::Switch, &o.help}};
}

// Fills `o` from argv; on a bad command line returns false with `err` set.
bool parse_options(int argc, char** argv, Options& o, std::string& err) {
    const std::vector<OptionSpec> specs = option_specs(o);
    for (int at = 1; at < argc; ++at) {
        const std::string arg = argv[at];
        if (arg == "-h") {
            o.help = true;
            continue;
        }
        if (arg.size() < 3 || arg.compare(0, 2, "--") != 0) {
            if (at != 1) {
                err = "unexpected argument '" + arg + "'";
                return false;
            }
            o.mode = arg;   // the mode comes first
            continue;
        }
        const size_t eq = arg.find('=');
        const std::string name = arg.substr(2, eq == std::string::npos ? std::string::npos : eq - 2);
        const auto spec = std::find_if(specs.begin(), specs.end(), [&](const OptionSpec& x) { return name == x.name; });
        if (spec == specs.end()) {
            err = "unknown option --" + name;
            return false;
        }
        if (spec->kind == OptionSpec::Switch) {
            if (eq != std::string::npos) {
                err = "--" + name + " takes no value";
                return false;
            }
            *static_cast<bool*>(spec->field) = true;
            continue;
        }
        std::string value;
        if (eq != std::string::npos) value = arg.substr(eq + 1);
        else if (at + 1 < argc) value = argv[++at];
        else {
            err = "--" + name + " needs a value";
            return false;
        }
        char* rest = nullptr;
        errno = 0;
        if (spec->kind == OptionSpec::Int) {
            const long x = std::strtol(value.c_str(), &rest, 10);
            if (errno || rest == value.c_str() || *rest || x < INT_MIN || x > INT_MAX) {
                err = "--" + name + " needs an integer, got '" + value + "'";
                return false;
            }
            *static_cast<int*>(spec->field) = static_cast<int>(x);
        } else if (spec->kind == OptionSpec::Real) {
            const double x = std::strtod(value.c_str(), &rest);
            if (errno || rest == value.c_str() || *rest) {
                err = "--" + name + " needs a number, got '" + value + "'";
                return false;
            }
            *static_cast<double*>(spec->field) = x;
        } else {
            *static_cast<std::string*>(spec->field) = value;
        }
    }
    if (!o.dtype.empty() && o.dtype != "fp16" && o.dtype != "fp8") {
        err = "--dtype must be fp16 or fp8";
        return false;
    }
    return true;
}

const char* kUsage =
    "usage: bench_decode sweep|ctas|pagesize|capacity|copy|single [--batch B] [--len L] [--dtype fp16|fp8]\n"
    "       [--hq 32] [--hkv 8] [--dim 128] [--page 16] [--iters 50] [--ctas 0] [--contiguous-pages]\n"
    "       [--budget-gib 1] [--max-len 8192] [--peak-gbps 8000|device]\n"
    "  --peak-gbps device: the device's memory clock x bus width x 2 (double data rate)\n";

// ---- timing -----------------------------------------------------------------

struct Flusher {   // 1 GiB streaming read between timed runs
    void*     buf  = nullptr;
    uint32_t* sink = nullptr;
    size_t    bytes = size_t{1} << 30;
    Flusher() {
        HIP_CHECK(hipMalloc(&buf, bytes));
        HIP_CHECK(hipMalloc(&sink, sizeof(uint32_t)));
        HIP_CHECK(hipMemset(buf, 1, bytes));
    }
    ~Flusher() {
        (void)hipFree(buf);
        (void)hipFree(sink);
    }
    void flush() const { decode::detail::check(pa_stream_read(buf, bytes, 2048, sink, nullptr)); }
};

// 5 flushed warm-ups, then `iters` runs each after a flush; median ms.
template <class F>
double time_cold(const Flusher* fl, int iters, F&& run) {
    hipEvent_t a, b;
    HIP_CHECK(hipEventCreate(&a));
    HIP_CHECK(hipEventCreate(&b));
    for (int w = 0; w < 5; ++w) {
        if (fl) fl->flush();
        run();
    }
    std::vector<float> ms;
    for (int it = 0; it < iters; ++it) {
        if (fl) fl->flush();
        HIP_CHECK(hipEventRecord(a, nullptr));
        run();
        HIP_CHECK(hipEventRecord(b, nullptr));
        HIP_CHECK(hipEventSynchronize(b));
        float m = 0;
        HIP_CHECK(hipEventElapsedTime(&m, a, b));
        ms.push_back(m);
    }
    HIP_CHECK(hipEventDestroy(a));
    HIP_CHECK(hipEventDestroy(b));
    std::sort(ms.begin(), ms.end());
    return ms.empty() ? 0.0 : ms[ms.size() / 2];
}

// ---- one decode configuration -------------------------------------------------

struct Shape {
    int batch, len, hq, hkv, dim, page;
    decode::KVDtype dtype;
    bool shuffle;
};

// bench_decode.cu:186-191: K and V once, q in and out once, the block table.
double algorithmic_bytes(const Shape& s) {
    const double e = decode::kv_dtype_bytes(s.dtype);
    const double pages = std::ceil(static_cast<double>(s.len) / s.page);
    return 2.0 * s.batch * s.len * s.hkv * s.dim * e + 2.0 * s.batch * s.hq * s.dim * 2 + s.batch * pages * 4;
}

// A Setup frees nothing before its destructor, and the multi-row modes keep
// every row's Setup until the mode ends: a row timed within some milliseconds
// of a large hipFree ran about 5% slower (32 x 8192 fp16: 170.8 against
// 161.7 us) while the freed memory was being released.
struct Setup {
    Shape shape;
    std::unique_ptr<decode::PagedKVCache> cache;
    __half* q   = nullptr;
    __half* out = nullptr;
    __half* k   = nullptr;   // source rows, kept until the destructor
    __half* v   = nullptr;

    explicit Setup(const Shape& s) : shape(s) {
        const int pages_per = (s.len + s.page - 1) / s.page;
        const size_t row = static_cast<size_t>(s.hkv) * s.dim;
        const size_t n = static_cast<size_t>(s.len) * row;
        HIP_CHECK(hipMalloc(&k, sizeof(__half) * n * s.batch));
        HIP_CHECK(hipMalloc(&v, sizeof(__half) * n * s.batch));
        hipLaunchKernelGGL(fill_normal_f16, dim3(4096), dim3(256), 0, 0, k, n * s.batch, 1u);
        hipLaunchKernelGGL(fill_normal_f16, dim3(4096), dim3(256), 0, 0, v, n * s.batch, 2u);
        HIP_CHECK(hipGetLastError());
        float k_scale = 1.0f, v_scale = 1.0f;
        if (s.dtype == decode::KVDtype::FP8_E4M3) {
            unsigned int* am = nullptr;
            HIP_CHECK(hipMalloc(&am, 2 * sizeof(unsigned int)));
            HIP_CHECK(hipMemset(am, 0, 2 * sizeof(unsigned int)));
            hipLaunchKernelGGL(abs_max_f16, dim3(2048), dim3(256), 0, 0, k, n * s.batch, am);
            hipLaunchKernelGGL(abs_max_f16, dim3(2048), dim3(256), 0, 0, v, n * s.batch, am + 1);
            unsigned int h[2];
            HIP_CHECK(hipMemcpy(h, am, sizeof(h), hipMemcpyDeviceToHost));
            HIP_CHECK(hipFree(am));
            float kmax, vmax;
            std::memcpy(&kmax, &h[0], 4);
            std::memcpy(&vmax, &h[1], 4);
            k_scale = kmax / 448.0f;
            v_scale = vmax / 448.0f;
        }
        decode::PagedKVCache::Config cfg{};
        cfg.num_pages          = s.batch * pages_per;
        cfg.page_size          = s.page;
        cfg.num_kv_heads       = s.hkv;
        cfg.head_dim           = s.dim;
        cfg.max_slots          = s.batch;
        cfg.max_pages_per_slot = pages_per;
        cfg.dtype              = s.dtype;
        cfg.k_scale            = k_scale;
        cfg.v_scale            = v_scale;
        cache = std::make_unique<decode::PagedKVCache>(cfg);
        if (s.shuffle) cache->shuffle_free_pages(42);
        for (int b = 0; b < s.batch; ++b) {
            const int slot = cache->admit();
            if (slot < 0 || !cache->append(slot, k + n * b, v + n * b, s.len))
                throw std::runtime_error("setup: the cache is full");
        }
        const size_t qn = static_cast<size_t>(s.batch) * s.hq * s.dim;
        HIP_CHECK(hipMalloc(&q, sizeof(__half) * qn));
        HIP_CHECK(hipMalloc(&out, sizeof(__half) * qn));
        hipLaunchKernelGGL(fill_normal_f16, dim3(256), dim3(256), 0, 0, q, qn, 3u);
        HIP_CHECK(hipDeviceSynchronize());
    }
    ~Setup() {
        (void)hipFree(q);
        (void)hipFree(out);
        (void)hipFree(k);
        (void)hipFree(v);
    }
    void plan(int ctas) {
        std::vector<int> slots(static_cast<size_t>(shape.batch));
        for (int b = 0; b < shape.batch; ++b) slots[static_cast<size_t>(b)] = b;
        cache->plan(slots, shape.hq, ctas);
    }
    void run() { cache->run(q, out); }
};

struct Gpu {
    std::string name;
    int cus = 0;
    double peak = 8000.0;
};

const char* kHeader = "gpu,dtype,batch,seq_len,hq,hkv,dim,page,ctas,segments,time_us,gbps,pct_peak";

void run_one(const Gpu& g, const Flusher& fl, Setup& s, int ctas, int iters) {
    s.plan(ctas);
    const double ms = time_cold(&fl, iters, [&] { s.run(); });
    const double gbps = algorithmic_bytes(s.shape) / (ms * 1e-3) / 1e9;
    const decode::DecodePlan& p = s.cache->last_plan();
    std::printf("%s,%s,%d,%d,%d,%d,%d,%d,%d,%zu,%.2f,%.1f,%.1f\n", g.name.c_str(),
                decode::kv_dtype_name(s.shape.dtype), s.shape.batch, s.shape.len, s.shape.hq, s.shape.hkv,
                s.shape.dim, s.shape.page, p.num_ctas, p.segments.size(), ms * 1e3, gbps, 100.0 * gbps / g.peak);
    std::fflush(stdout);
}

int run(const Options& a) {
    Gpu g;
    {
        hipDeviceProp_t prop;
        int dev = 0;
        HIP_CHECK(hipGetDevice(&dev));
        HIP_CHECK(hipGetDeviceProperties(&prop, dev));
        g.name = prop.name;
        if (g.name.empty() || g.name == "AMD Radeon Graphics") {   // the marketing name needs libdrm's id
                                                                    // table; fall back to the ISA name
            const std::string arch = prop.gcnArchName;
            g.name = "AMD " + arch.substr(0, arch.find(':'));
        }
        std::replace(g.name.begin(), g.name.end(), ',', ' ');
        g.cus = prop.multiProcessorCount;
        // The DRAM peak the device reports (bench_decode.cu:87-100 derives it
        // the same way): memory clock (kHz) x bus width (bits) / 8 x 2.
        int clock_khz = 0, bus_bits = 0;
        if (hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeMemoryClockRate, dev) != hipSuccess) clock_khz = 0;
        if (hipDeviceGetAttribute(&bus_bits, hipDeviceAttributeMemoryBusWidth, dev) != hipSuccess) bus_bits = 0;
        const double device_peak = 2.0 * clock_khz * 1e3 * (bus_bits / 8.0) / 1e9;
        std::fprintf(stderr, "# device-reported DRAM peak: %.0f GB/s (memory clock %d kHz, bus %d bits)\n",
                     device_peak, clock_khz, bus_bits);
        if (a.peak == "device") {
            if (device_peak <= 0) throw std::runtime_error("the device reports no memory clock or bus width");
            g.peak = device_peak;
        } else {
            char* rest = nullptr;
            g.peak = std::strtod(a.peak.c_str(), &rest);
            if (rest == a.peak.c_str() || *rest || g.peak <= 0)
                throw std::invalid_argument("--peak-gbps needs a positive number or 'device'");
        }
    }
    std::fprintf(stderr, "# %s, %d CUs, HBM peak %.0f GB/s\n", g.name.c_str(), g.cus, g.peak);
    const int hq = a.hq, hkv = a.hkv, dim = a.dim;
    const int page = a.page, iters = a.iters, ctas = a.ctas;
    const bool shuffle = !a.contiguous_pages;
    const decode::KVDtype dt = a.dtype == "fp8" ? decode::KVDtype::FP8_E4M3 : decode::KVDtype::FP16;

    if (a.mode == "copy") {   // bench_decode.cu:224-240 plus the chunked read
        const size_t bytes = size_t{4} << 30;
        void* buf = nullptr;
        uint32_t* sink = nullptr;
        HIP_CHECK(hipMalloc(&buf, bytes));
        HIP_CHECK(hipMalloc(&sink, sizeof(uint32_t)));
        HIP_CHECK(hipMemset(buf, 1, bytes));
        std::printf("gpu,kernel,bytes,time_us,gbps,pct_peak\n");
        auto row = [&](const std::string& name, double ms) {
            const double gbps = bytes / (ms * 1e-3) / 1e9;
            std::printf("%s,%s,%zu,%.2f,%.1f,%.1f\n", g.name.c_str(), name.c_str(), bytes, ms * 1e3, gbps,
                        100.0 * gbps / g.peak);
            std::fflush(stdout);
        };
        for (int mult : {4, 8, 16, 32}) {
            const int blocks = g.cus * mult;
            row("read_" + std::to_string(blocks) + "x512", time_cold(nullptr, 10, [&] {
                    decode::detail::check(pa_stream_read_ex(buf, bytes, blocks, 512, 1, 0, sink, nullptr));
                }));
        }
        for (auto [mult, unroll] : {std::pair<int, int>{1, 16}, {2, 16}, {4, 8}}) {
            const int blocks = g.cus * mult;
            if (bytes % (static_cast<size_t>(blocks) * 8 * unroll * 1024) != 0) continue;
            row("read_chunked_" + std::to_string(blocks) + "x512_u" + std::to_string(unroll) + "_nt",
                time_cold(nullptr, 10, [&] {
                    decode::detail::check(pa_stream_read_chunked(buf, bytes, blocks, 512, unroll, sink, nullptr));
                }));
        }
        HIP_CHECK(hipFree(buf));
        HIP_CHECK(hipFree(sink));
        return 0;
    }
    if (a.mode == "capacity") {   // bench_decode.cu:285-321 through the host allocator
        const size_t budget = static_cast<size_t>(a.budget_gib * static_cast<double>(size_t{1} << 30));
        const int max_len = a.max_len;
        const int per_slot = (max_len + page - 1) / page;
        std::printf("dtype,layout,max_len,actual_len,sequences,bytes_per_seq\n");
        for (int actual : {256, 512, 1024, 2048, 4096, 8192}) {
            const size_t contiguous = 2ull * max_len * hkv * dim * 2;
            std::printf("fp16,contiguous,%d,%d,%zu,%zu\n", max_len, actual, budget / contiguous, contiguous);
            for (decode::KVDtype kd : {decode::KVDtype::FP16, decode::KVDtype::FP8_E4M3}) {
                decode::PagedKVCache::Config cfg{};
                cfg.page_size = page;
                cfg.num_kv_heads = hkv;
                cfg.head_dim = dim;
                cfg.max_pages_per_slot = per_slot;
                cfg.dtype = kd;
                const int pages = decode::PagedKVCache::pages_for_budget(cfg, budget);
                pa_pool* pool = nullptr;
                decode::detail::check(pa_pool_create(pages, page, pages, per_slot, &pool));
                int n = 0;
                for (;;) {
                    const int slot = pa_pool_admit(pool);
                    int ok = 0, first = 0, num = 0;
                    if (slot < 0) break;
                    decode::detail::check(pa_pool_reserve(pool, slot, actual, &ok, &first, &num));
                    if (!ok) break;
                    ++n;
                }
                pa_pool_destroy(pool);
                const size_t total = decode::PagedKVCache::bytes_per_page(cfg) * static_cast<size_t>(pages);
                std::printf("%s,paged,%d,%d,%d,%zu\n", decode::kv_dtype_name(kd), max_len, actual, n,
                            n ? total / static_cast<size_t>(n) : 0);
            }
        }
        return 0;
    }

    Flusher fl;
    const int batch = a.batch, len = a.len;
    if (a.mode == "sweep") {
        std::printf("%s\n", kHeader);
        std::vector<decode::KVDtype> dts;
        if (!a.dtype.empty()) dts = {dt};
        else dts = {decode::KVDtype::FP16, decode::KVDtype::FP8_E4M3};
        const std::vector<std::pair<int, int>> shapes = {{1, 4096},  {1, 16384}, {1, 65536}, {1, 131072},
                                                         {8, 4096},  {8, 16384}, {8, 32768}, {32, 1024},
                                                         {32, 4096}, {32, 8192}, {64, 1024}, {64, 4096},
                                                         {128, 1024}, {128, 2048}};
        std::vector<std::unique_ptr<Setup>> kept;
        for (decode::KVDtype d : dts)
            for (auto [b, l] : shapes) {
                kept.push_back(std::make_unique<Setup>(Shape{b, l, hq, hkv, dim, page, d, shuffle}));
                run_one(g, fl, *kept.back(), ctas, iters);
            }
        return 0;
    }
    if (a.mode == "single") {
        std::printf("%s\n", kHeader);
        Setup s(Shape{batch, len, hq, hkv, dim, page, dt, shuffle});
        run_one(g, fl, s, ctas, iters);
        return 0;
    }
    if (a.mode == "ctas") {
        std::printf("%s\n", kHeader);
        Setup s(Shape{batch, len, hq, hkv, dim, page, dt, shuffle});
        const int wave = decode::wave_ctas(dt, dim, hq / hkv);
        std::fprintf(stderr, "# one wave = %d work units\n", wave);
        std::vector<int> grid = {g.cus / 2, g.cus, 2 * g.cus, 3 * g.cus, 4 * g.cus, 6 * g.cus,
                                 8 * g.cus, 12 * g.cus, 16 * g.cus, wave};
        std::sort(grid.begin(), grid.end());
        grid.erase(std::unique(grid.begin(), grid.end()), grid.end());
        for (int n : grid) run_one(g, fl, s, n, iters);
        return 0;
    }
    if (a.mode == "pagesize") {
        std::printf("%s\n", kHeader);
        std::vector<std::unique_ptr<Setup>> kept;
        for (int ps : {1, 4, 8, 16, 32, 64, 128, 256, 1024, len}) {
            if (ps > len) continue;
            kept.push_back(std::make_unique<Setup>(Shape{batch, len, hq, hkv, dim, ps, dt, shuffle}));
            run_one(g, fl, *kept.back(), ctas, iters);
        }
        return 0;
    }
    std::fprintf(stderr, "unknown mode %s\n%s", a.mode.c_str(), kUsage);
    return 1;
}

}  // namespace

int main(int argc, char** argv) {
    Options a;
    std::string err;
    if (!parse_options(argc, argv, a, err)) {   // no device use
        std::fprintf(stderr, "bench_decode: %s\n%s", err.c_str(), kUsage);
        return 2;
    }
    if (a.help || a.mode == "help") {
        std::fputs(kUsage, stdout);
        return 0;
    }
    static const char* const kModes[] = {"sweep", "ctas", "pagesize", "capacity", "copy", "single"};
    if (std::none_of(std::begin(kModes), std::end(kModes), [&](const char* m) { return a.mode == m; })) {
        std::fprintf(stderr, "bench_decode: unknown mode %s\n%s", a.mode.c_str(), kUsage);
        return 2;
    }
    try {
        return run(a);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "bench_decode: %s\n", e.what());
        return 1;
    }
}
