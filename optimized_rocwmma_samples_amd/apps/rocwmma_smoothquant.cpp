// rocwmma_smoothquant -- SmoothQuant fp16 -> int8 row quantization on MI355X.
// Command line and result line of the reference sample
// (rocwmma_smoothquant.cpp:166-176): `rocwmma_smoothquant [M N]`, default
// 3328 x 4096, then N in {1024, 2048, 8192};
//   [SmoothQuant] M=<M> N=<N>  <ms> ms  <GB/s> GB/s
// with the reference's bytes formula (2MN + MN + 4N + 4M, :157-158).  Inputs
// are seeded N(0,1) activations with 0.5% x20 outlier columns and a U[0.5, 2]
// smooth scale (the reference fills constants, :140-141).
#include "common.hpp"

static void test_smoothquant(uint32_t M, uint32_t N, bool verify)
{
    const uint64_t seed = app::config_seed(1);
    auto           hx   = app::gen_activations(seed, M, N);
    auto           hs   = app::gen_uniform(seed, app::kS, N, 0.5, 2.0);
    app::Dev<uint16_t> dx(hx);
    app::Dev<float>    ds(hs);
    app::Dev<int8_t>   dq((size_t)M * N);
    app::Dev<float>    dr(M);
    auto fn = [&] {
        CHECK_W8A8(w8a8_smoothquant(dx.p, ds.p, dq.p, dr.p, M, N, 127.f, 0, 0, nullptr));
    };
    const double ms = app::bench_ms(fn);
    const double bw = ((double)M * N * 2 + (double)M * N + 4.0 * N + 4.0 * M) / (ms * 1e-3) / 1e9;
    std::cout << "[SmoothQuant] M=" << M << " N=" << N << "  " << ms << " ms  " << bw << " GB/s\n";
    if(verify) {
        std::vector<int8_t> q((size_t)M * N);
        std::vector<float>  r(M);
        app::cpu_smoothquant(hx.data(), hs.data(), q.data(), r.data(), M, N, 127.f);
        const auto   gq   = dq.download();
        const auto   gr   = dr.download();
        size_t       bad  = 0;
        for(size_t i = 0; i < q.size(); ++i) bad += gq[i] != q[i];
        size_t badr = 0;
        for(size_t i = 0; i < r.size(); ++i) badr += std::memcmp(&gr[i], &r[i], 4) != 0;
        app::report(bad == 0 && badr == 0, "q mismatches=" + std::to_string(bad) +
                                               " row-scale mismatches=" + std::to_string(badr));
    }
}

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(argc, argv, "rocwmma_smoothquant [M N] [--verify]");
    const auto         d = app::sizes(o, {2});
    uint32_t           M = 3328, N = 4096;
    if(!d.empty()) {
        M = d[0];
        N = d[1];
    }
    app::banner("W8A8 SmoothQuant (MI355X gfx950)");
    test_smoothquant(M, N, o.verify);
    for(uint32_t n : {1024u, 2048u, 8192u}) test_smoothquant(M, n, o.verify);
    return 0;
}
