// rocwmma_rmsnorm2d -- RMSNorm, Add+RMSNorm and Add+RMSNorm fused with the
// SmoothQuant quantizer on MI355X.
// Command line and result lines of the reference sample
// (rocwmma_rmsnorm2d.cpp:255-265): `rocwmma_rmsnorm2d [M N]`, default
// 3328 x 4096, then RMSNorm at N in {1024, 2048, 8192}:
//   [RMSNorm2D] M=<M> N=<N>  <ms> ms  <GB/s> GB/s        bytes 2*2MN + 4N (:219)
//   [Add+RMSNorm2D] M=<M> N=<N>  <ms> ms  <GB/s> GB/s    bytes 4*2MN + 4N (:247)
// plus the fused form this library adds (x + residual -> x_out, then int8 +
// row scale without writing y):
//   [Add+RMSNorm2D+SQ] M=<M> N=<N>  <ms> ms  <GB/s> GB/s bytes 3*2MN + MN + 4M + 8N
// eps = 1e-5 as in the reference.  Inputs are seeded (the reference fills
// constants, :204-205, :228-229): activation-like x, N(0,1) residual, gamma
// U[0.5, 1.5], smooth scale U[0.5, 2].
#include "common.hpp"

namespace {

constexpr float kEps = 1e-5f;

struct Inputs {
    std::vector<uint16_t> x, res;
    std::vector<float>    gamma, s;
};

Inputs make_inputs(uint32_t M, uint32_t N)
{
    const uint64_t seed = app::config_seed(3) ^ 0x4E;
    Inputs         in;
    in.x     = app::gen_activations(seed, M, N);
    auto r   = app::gen_normal(seed, app::kResidual, (size_t)M * N);
    in.res.resize(r.size());
    for(size_t i = 0; i < r.size(); ++i) in.res[i] = app::f2h(r[i]);
    in.gamma = app::gen_uniform(seed, app::kGamma, N, 0.5, 1.5);
    in.s     = app::gen_uniform(seed, app::kS, N, 0.5, 2.0);
    return in;
}

// CPU restatement: v = x (+ res) in fp32, x_out = half(v), sum of squares in
// float64, rstd = 1/sqrt(sum/N + eps), y = half((u * rstd) * gamma) with u the
// saved half(v) when there is a residual (rocwmma_rmsnorm2d.cpp:156-182).
void cpu_rmsnorm(const Inputs& in, bool with_res, uint32_t M, uint32_t N,
                 std::vector<uint16_t>& xo, std::vector<uint16_t>& y)
{
    xo.assign((size_t)M * N, 0);
    y.assign((size_t)M * N, 0);
#pragma omp parallel for
    for(size_t m = 0; m < M; ++m) {
        std::vector<float> v(N);
        double             ss = 0.0;
        for(size_t n = 0; n < N; ++n) {
            v[n] = app::h2f(in.x[m * N + n]);
            if(with_res) v[n] += app::h2f(in.res[m * N + n]);
            ss += (double)v[n] * (double)v[n];
        }
        const float mean = (float)ss / (float)N;
        const float rstd = (float)(1.0 / std::sqrt((double)(mean + kEps)));
        for(size_t n = 0; n < N; ++n) {
            float u = v[n];
            if(with_res) {
                xo[m * N + n] = app::f2h(v[n]);
                u             = app::h2f(xo[m * N + n]);
            }
            y[m * N + n] = app::f2h((u * rstd) * in.gamma[n]);
        }
    }
}

// fp16 ulp distance
int ulps(uint16_t a, uint16_t b)
{
    auto key = [](uint16_t h) { return (h & 0x8000) ? -(int)(h & 0x7FFF) : (int)h; };
    return std::abs(key(a) - key(b));
}

void check_y(const std::vector<uint16_t>& got, const std::vector<uint16_t>& exp, const char* what)
{
    size_t off = 0, far = 0;
    for(size_t i = 0; i < got.size(); ++i) {
        const int d = ulps(got[i], exp[i]);
        off += d > 0;
        far += d > 1;
    }
    app::report(far == 0 && off <= std::max<size_t>(2, got.size() / 100),
                std::string(what) + " y: " + std::to_string(off) + " of " +
                    std::to_string(got.size()) + " one ulp off, " + std::to_string(far) +
                    " further");
}

void test_rmsnorm(uint32_t M, uint32_t N, bool verify)
{
    const Inputs       in = make_inputs(M, N);
    app::Dev<uint16_t> dx(in.x), dy((size_t)M * N);
    app::Dev<float>    dg(in.gamma);
    auto fn = [&] {
        CHECK_W8A8(w8a8_add_rmsnorm_smoothquant(dx.p, nullptr, dg.p, nullptr, nullptr, dy.p,
                                                nullptr, nullptr, M, N, kEps, 127.f, 0, 0, 0,
                                                nullptr));
    };
    const double ms = app::bench_ms(fn);
    const double bw = ((double)M * N * 2.0 * 2 + 4.0 * N) / (ms * 1e-3) / 1e9;
    std::cout << "[RMSNorm2D] M=" << M << " N=" << N << "  " << ms << " ms  " << bw << " GB/s\n";
    if(verify) {
        std::vector<uint16_t> xo, y;
        cpu_rmsnorm(in, false, M, N, xo, y);
        check_y(dy.download(), y, "RMSNorm2D");
    }
}

void test_add_rmsnorm(uint32_t M, uint32_t N, bool verify, bool fused_sq)
{
    const Inputs       in = make_inputs(M, N);
    app::Dev<uint16_t> dx(in.x), dr(in.res), dxo((size_t)M * N), dy((size_t)M * N);
    app::Dev<float>    dg(in.gamma), ds(in.s), drs(M);
    app::Dev<int8_t>   dq((size_t)M * N);
    auto fn = [&] {
        if(fused_sq)
            CHECK_W8A8(w8a8_add_rmsnorm_smoothquant(dx.p, dr.p, dg.p, ds.p, dxo.p, nullptr, dq.p,
                                                    drs.p, M, N, kEps, 127.f, 0, 0, 0, nullptr));
        else
            CHECK_W8A8(w8a8_add_rmsnorm_smoothquant(dx.p, dr.p, dg.p, nullptr, dxo.p, dy.p,
                                                    nullptr, nullptr, M, N, kEps, 127.f, 0, 0, 0,
                                                    nullptr));
    };
    const double ms    = app::bench_ms(fn);
    const double bytes = fused_sq ? (double)M * N * 7.0 + 4.0 * M + 8.0 * N
                                  : (double)M * N * 4.0 * 2 + 4.0 * N;
    std::cout << (fused_sq ? "[Add+RMSNorm2D+SQ] M=" : "[Add+RMSNorm2D] M=") << M << " N=" << N
              << "  " << ms << " ms  " << bytes / (ms * 1e-3) / 1e9 << " GB/s\n";
    if(verify) {
        std::vector<uint16_t> xo, y;
        cpu_rmsnorm(in, true, M, N, xo, y);
        const auto gxo = dxo.download();
        size_t     bad = 0;
        for(size_t i = 0; i < xo.size(); ++i) bad += gxo[i] != xo[i];
        app::report(bad == 0, "x_out mismatches=" + std::to_string(bad));
        if(!fused_sq) {
            check_y(dy.download(), y, "Add+RMSNorm2D");
            return;
        }
        // the quantized row must be the quantizer's output for a y within one
        // ulp of the CPU's: |q diff| <= 1, row scales within 2e-3
        std::vector<int8_t> q((size_t)M * N);
        std::vector<float>  r(M);
        app::cpu_smoothquant(y.data(), in.s.data(), q.data(), r.data(), M, N, 127.f);
        const auto gq = dq.download();
        const auto gr = drs.download();
        size_t     qoff = 0, qfar = 0, rfar = 0;
        for(size_t i = 0; i < q.size(); ++i) {
            const int d = std::abs((int)gq[i] - (int)q[i]);
            qoff += d > 0;
            qfar += d > 1;
        }
        for(size_t i = 0; i < r.size(); ++i)
            rfar += std::fabs(gr[i] - r[i]) > 2e-3f * std::fabs(r[i]);
        app::report(qfar == 0 && rfar == 0, "q: " + std::to_string(qoff) + " off by one, " +
                                                std::to_string(qfar) + " further; row scales off: " +
                                                std::to_string(rfar));
    }
}

} // namespace

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(argc, argv, "rocwmma_rmsnorm2d [M N] [--verify]");
    const auto         d = app::sizes(o, {2});
    uint32_t           M = 3328, N = 4096;
    if(!d.empty()) {
        M = d[0];
        N = d[1];
    }
    app::banner("W8A8 RMSNorm2D / Add+RMSNorm2D (+ SmoothQuant) (MI355X gfx950)");
    test_rmsnorm(M, N, o.verify);
    test_add_rmsnorm(M, N, o.verify, false);
    test_add_rmsnorm(M, N, o.verify, true);
    for(uint32_t n : {1024u, 2048u, 8192u}) test_rmsnorm(M, n, o.verify);
    return 0;
}
