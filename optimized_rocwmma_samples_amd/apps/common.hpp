// common.hpp -- shared host code of the sample CLIs: error checks, timing,
// seeded inputs, device banner, and the CPU verification the Debug build runs.
//
// The CLIs keep the reference samples' command lines and result lines
// ("[Label] ... <ms> ms  <x> GB/s | TFlops/s", parsed by benchmark.sh:180-187)
// and their Debug-build CPU check (rocwmma_perf_gemm.cpp:736-749: a build
// without NDEBUG verifies).  Here the check is on when the CLI is built with
// `build.py --debug` (W8A8_CPU_VERIFY), or at run time with --verify or
// W8A8_VERIFY=1.  Inputs are seeded (the counter-based generator of
// optimized_rocwmma_samples_amd/datagen.py), so every run sees the same data.
#pragma once

#include "../../include/w8a8.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <iostream>
#include <memory>
#include <string>
#include <vector>

#define CHECK_HIP(cmd)                                                                      \
    do {                                                                                    \
        hipError_t e_ = (cmd);                                                              \
        if(e_ != hipSuccess) {                                                              \
            std::cerr << "HIP " << hipGetErrorString(e_) << " at " << __FILE__ << ":"      \
                      << __LINE__ << "\n";                                                  \
            std::exit(1);                                                                   \
        }                                                                                   \
    } while(0)

#define CHECK_W8A8(cmd)                                                                     \
    do {                                                                                    \
        int s_ = (cmd);                                                                     \
        if(s_ != W8A8_SUCCESS) {                                                            \
            std::cerr << #cmd << " -> " << s_ << ": " << w8a8_last_error() << "\n";         \
            std::exit(1);                                                                   \
        }                                                                                   \
    } while(0)

namespace app {

// ---------------------------------------------------------------- options
// Command line of a CLI: positional sizes (the reference's `[M N K]`
// grammar), --verify / --no-verify, -h / --help, and the CLI's own extra
// flags.  Every check here runs before the first HIP call, so argument errors
// end with status 1 and a usage line on any host, GPU or not.
struct Options {
    bool                     verify = false;
    std::vector<std::string> pos;   // positional arguments
    std::vector<std::string> flags; // extra flags given (from the CLI's list), "--name=value" whole
    const char*              usage = "";
    bool has(const char* f) const { return std::find(flags.begin(), flags.end(), f) != flags.end(); }
    // value of "--name=value" for an extra flag listed as "--name="; nullptr if absent
    const char* value(const char* f) const
    {
        const std::string pre = f;
        for(const std::string& g : flags)
            if(g.compare(0, pre.size(), pre) == 0) return g.c_str() + pre.size();
        return nullptr;
    }
};

[[noreturn]] inline void usage_error(const Options& o, const std::string& msg)
{
    std::cerr << "[ERROR] " << msg << "\nusage: " << o.usage << "\n";
    std::exit(1);
}

inline Options parse(int argc, char** argv, const char* usage,
                     std::initializer_list<const char*> extra = {})
{
    Options o;
    o.usage = usage;
#if defined(W8A8_CPU_VERIFY)
    o.verify = true;
#endif
    if(const char* v = std::getenv("W8A8_VERIFY")) o.verify = o.verify || std::atoi(v) != 0;
    for(int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if(a == "-h" || a == "--help") {
            std::cout << "usage: " << usage << "\n";
#if defined(W8A8_CPU_VERIFY)
            std::cout << "CPU verify: on by default (debug build; --no-verify turns it off)\n";
#else
            std::cout << "CPU verify: off by default (--verify or W8A8_VERIFY=1 turns it on)\n";
#endif
            std::exit(0);
        } else if(a == "--verify") {
            o.verify = true;
        } else if(a == "--no-verify") {
            o.verify = false;
        } else if(a.size() > 1 && a[0] == '-') {
            bool known = false;
            for(const char* f : extra) {
                const std::string e = f;
                known = known || a == e
                        || (!e.empty() && e.back() == '=' && a.compare(0, e.size(), e) == 0);
            }
            if(!known) usage_error(o, "unknown option " + a);
            o.flags.push_back(a);
        } else {
            o.pos.push_back(a);
        }
    }
    return o;
}

// The positional sizes: none (the CLI runs its default suite) or exactly one
// of the allowed counts, each a decimal integer in [1, 2^31).
inline std::vector<uint32_t> sizes(const Options& o, std::initializer_list<size_t> counts)
{
    if(o.pos.empty()) return {};
    bool ok = false;
    for(size_t c : counts) ok = ok || o.pos.size() == c;
    if(!ok) usage_error(o, "wrong number of sizes (" + std::to_string(o.pos.size()) + ")");
    std::vector<uint32_t> v;
    for(const std::string& a : o.pos) {
        char*              end = nullptr;
        errno                  = 0;
        const long long    x   = std::strtoll(a.c_str(), &end, 10);
        if(a.empty() || *end != '\0' || errno != 0 || x < 1 || x >= (1ll << 31))
            usage_error(o, "size '" + a + "' is not an integer in [1, 2^31)");
        v.push_back((uint32_t)x);
    }
    return v;
}

inline void banner(const char* title)
{
    hipDeviceProp_t prop;
    CHECK_HIP(hipGetDeviceProperties(&prop, 0));
    std::cout << "Device: " << prop.name << "  (" << prop.gcnArchName << ")\n\n";
    std::cout << "=== " << title << " ===\n";
}

// ms per run: `warmup` untimed launches, then `runs` back to back between events
template <class F>
double bench_ms(F fn, int warmup = 5, int runs = 20)
{
    for(int i = 0; i < warmup; ++i) fn();
    CHECK_HIP(hipDeviceSynchronize());
    hipEvent_t t0, t1;
    CHECK_HIP(hipEventCreate(&t0));
    CHECK_HIP(hipEventCreate(&t1));
    CHECK_HIP(hipEventRecord(t0, 0));
    for(int i = 0; i < runs; ++i) fn();
    CHECK_HIP(hipEventRecord(t1, 0));
    CHECK_HIP(hipEventSynchronize(t1));
    float ms = 0.f;
    CHECK_HIP(hipEventElapsedTime(&ms, t0, t1));
    CHECK_HIP(hipEventDestroy(t0));
    CHECK_HIP(hipEventDestroy(t1));
    return ms / runs;
}

// ------------------------------------------------------------ device memory
template <class T>
struct Dev {
    T*     p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) { CHECK_HIP(hipMalloc(&p, std::max<size_t>(1, n) * sizeof(T))); }
    Dev(const std::vector<T>& h) : Dev(h.size()) { upload(h); }
    ~Dev() { (void)hipFree(p); }
    Dev(const Dev&) = delete;
    Dev& operator=(const Dev&) = delete;
    void upload(const std::vector<T>& h)
    {
        CHECK_HIP(hipMemcpy(p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    }
    std::vector<T> download() const
    {
        std::vector<T> h(n);
        CHECK_HIP(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost));
        return h;
    }
};

// ---------------------------------------------------------- seeded inputs
// h(seed, tid, i) = splitmix64 finalizer of (seed ^ tid << 56) + (i + 1) * golden
enum Tid : uint64_t {
    kX = 1, kS = 2, kOutlier = 3, kA = 4, kB = 5, kSa = 6, kSb = 7, kLogits = 8, kExpertS = 9,
    kWDown = 10, kSbDown = 11, kResidual = 12, kGamma = 13
};

inline uint64_t h64(uint64_t seed, uint64_t tid, uint64_t i)
{
    uint64_t z = (seed ^ (tid << 56)) + (i + 1) * 0x9E3779B97F4A7C15ull;
    z          = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z          = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
inline double u01(uint64_t h) { return (double)(h >> 11) * 0x1.0p-53; }

inline uint16_t f2h(float f)
{
    _Float16 h = (_Float16)f; // round to nearest even
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}
inline float h2f(uint16_t b)
{
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (float)h;
}

inline std::vector<int8_t> gen_int8(uint64_t seed, uint64_t tid, size_t n)
{
    std::vector<int8_t> v(n);
#pragma omp parallel for
    for(size_t i = 0; i < n; ++i) v[i] = (int8_t)((int)(h64(seed, tid, i) % 255u) - 127);
    return v;
}

inline std::vector<float> gen_uniform(uint64_t seed, uint64_t tid, size_t n, double lo, double hi)
{
    std::vector<float> v(n);
#pragma omp parallel for
    for(size_t i = 0; i < n; ++i) v[i] = (float)(lo + (hi - lo) * u01(h64(seed, tid, i)));
    return v;
}

inline float normal_at(uint64_t seed, uint64_t tid, size_t i)
{
    const double u1 = 1.0 - u01(h64(seed, tid, 2 * i));
    const double u2 = u01(h64(seed, tid, 2 * i + 1));
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2));
}

inline std::vector<float> gen_normal(uint64_t seed, uint64_t tid, size_t n)
{
    std::vector<float> v(n);
#pragma omp parallel for
    for(size_t i = 0; i < n; ++i) v[i] = normal_at(seed, tid, i);
    return v;
}

// fp16 [m, k] N(0,1) activations with round(frac*k) outlier columns scaled x20
inline std::vector<uint16_t> gen_activations(uint64_t seed, size_t m, size_t k,
                                             double frac = 0.005, double scale = 20.0)
{
    const size_t          count = (size_t)std::llround(frac * (double)k);
    std::vector<uint64_t> perm(k);
    for(size_t j = 0; j < k; ++j) perm[j] = j;
    for(size_t j = 0; j < count; ++j) { // seeded partial Fisher-Yates
        const size_t r = j + (size_t)(h64(seed, kOutlier, j) % (uint64_t)(k - j));
        std::swap(perm[j], perm[r]);
    }
    std::vector<char> out_col(k, 0);
    for(size_t j = 0; j < count; ++j) out_col[perm[j]] = 1;
    std::vector<uint16_t> v(m * k);
#pragma omp parallel for
    for(size_t r = 0; r < m; ++r)
        for(size_t c = 0; c < k; ++c) {
            double z = normal_at(seed, kX, r * k + c);
            if(out_col[c]) z *= scale;
            v[r * k + c] = f2h((float)z);
        }
    return v;
}

inline uint64_t config_seed(int cfg) { return 0x5EED0000ull + (uint64_t)cfg; }

// ------------------------------------------------------- CPU verification
// SmoothQuant rows: p = x*s, r = max|p|/qmax, inv = r>0 ? 1/r : 0,
// q = clamp(rint(p*inv)) -- the reference's order (rocwmma_smoothquant.cpp:84-120).
inline void cpu_smoothquant(const uint16_t* x, const float* s, int8_t* q, float* r, size_t m,
                            size_t n, float qmax)
{
#pragma omp parallel for
    for(size_t i = 0; i < m; ++i) {
        float amax = 0.f;
        for(size_t j = 0; j < n; ++j) amax = std::max(amax, std::fabs(h2f(x[i * n + j]) * s[j]));
        const float rs  = amax / qmax;
        const float inv = rs > 0.f ? 1.f / rs : 0.f;
        r[i]            = rs;
        for(size_t j = 0; j < n; ++j) {
            const float v = (h2f(x[i * n + j]) * s[j]) * inv;
            q[i * n + j]  = (int8_t)std::min(std::max(std::nearbyint(v), -qmax), qmax);
        }
    }
}

// acc[i, j] = sum_h a[i, h] * b[j, h] (A [m, k] row-major, B [n, k]), rows of `rows`
inline std::vector<int32_t> cpu_gemm_i32(const int8_t* a, const int8_t* b, size_t m, size_t n,
                                         size_t k, const std::vector<size_t>& rows)
{
    std::vector<int32_t> c(rows.size() * n);
#pragma omp parallel for
    for(size_t ri = 0; ri < rows.size(); ++ri) {
        const int8_t* ar = a + rows[ri] * k;
        for(size_t j = 0; j < n; ++j) {
            const int8_t* br  = b + j * k;
            int32_t       acc = 0;
            for(size_t h = 0; h < k; ++h) acc += (int32_t)ar[h] * (int32_t)br[h];
            c[ri * n + j] = acc;
        }
    }
    (void)m;
    return c;
}

inline uint16_t cpu_dequant(int32_t acc, float sa, float sb) { return f2h(((float)acc * sa) * sb); }

// rows to check: all (m <= limit) or first, last and a spread of the rest
inline std::vector<size_t> sample_rows(size_t m, size_t limit = 512)
{
    std::vector<size_t> rows;
    if(m <= limit) {
        for(size_t i = 0; i < m; ++i) rows.push_back(i);
        return rows;
    }
    for(size_t i = 0; i < limit; ++i) rows.push_back(i * (m - 1) / (limit - 1));
    rows.erase(std::unique(rows.begin(), rows.end()), rows.end());
    return rows;
}

inline void report(bool ok, const std::string& what)
{
    std::cout << "  " << (ok ? "PASSED" : "FAILED") << "  " << what << "\n";
    if(!ok) std::exit(2);
}

} // namespace app
