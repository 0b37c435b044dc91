// rocwmma_streamk_gemm -- stream-K W8A8 GEMM on MI355X (w8a8_gemm_streamk).
// Stands in for the reference's stream-K sample (rocwmma_streamk_gemm.cpp:213-297):
// one block per CU, the problem's k-tiles cut into equal contiguous ranges,
// a tile shared by several blocks summed in int32 by the last of them to
// finish, in one launch (the reference flushes fp32 partials with atomics
// and reduces them in a second launch, :129-143, :185-211).
// `rocwmma_streamk_gemm [M N K] [--blocks=B]`; default: the reference's
// sizes (:286-297), 512^2 ... 4096^2 at K = 4096.  Result line
//   [StreamK-GEMM] M=<M> N=<N> K=<K> num_cus=<blocks launched>  <ms> ms  <TF> TFlops/s
#include "common.hpp"

static void test_streamk(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks, bool verify)
{
    const uint64_t seed = app::config_seed(4);
    auto           ha   = app::gen_int8(seed, app::kA, (size_t)m * k);
    auto           hw   = app::gen_int8(seed, app::kB, (size_t)n * k);
    auto           hsa  = app::gen_uniform(seed, app::kSa, m, 1e-3, 1e-2);
    auto           hsb  = app::gen_uniform(seed, app::kSb, n, 1e-3, 1e-2);
    app::Dev<int8_t>   da(ha), dw(hw);
    app::Dev<float>    dsa(hsa), dsb(hsb);
    app::Dev<uint16_t> dc((size_t)m * n);
    const size_t       wsb = w8a8_gemm_streamk_workspace_size(m, n, k, blocks);
    app::Dev<int8_t>   ws(std::max<size_t>(wsb, 16));
    auto fn = [&](void* c, int out) {
        CHECK_W8A8(w8a8_gemm_streamk(m, n, k, da.p, dw.p, c, k, k, n, dsa.p, dsb.p, 1.f, 1.f, out,
                                     blocks, ws.p, wsb, nullptr));
    };
    const double ms = app::bench_ms([&] { fn(dc.p, W8A8_OUT_F16); });
    std::cout << "[StreamK-GEMM] M=" << m << " N=" << n << " K=" << k
              << " num_cus=" << w8a8_gemm_streamk_blocks(m, n, k, blocks) << "  " << ms << " ms  "
              << 2.0 * m * n * k / (ms * 1e-3) / 1e12 << " TFlops/s\n";
    if(verify) {
        app::Dev<int32_t> di((size_t)m * n);
        fn(di.p, W8A8_OUT_I32);
        const auto rows = app::sample_rows(m, 64);
        const auto acc  = app::cpu_gemm_i32(ha.data(), hw.data(), m, n, k, rows);
        const auto gi   = di.download();
        const auto gc   = dc.download();
        size_t     bad  = 0;
        for(size_t ri = 0; ri < rows.size(); ++ri)
            for(size_t j = 0; j < n; ++j) {
                bad += gi[rows[ri] * n + j] != acc[ri * n + j];
                bad += gc[rows[ri] * n + j] != app::cpu_dequant(acc[ri * n + j], hsa[rows[ri]], hsb[j]);
            }
        uint32_t flags = 0;
        CHECK_W8A8(w8a8_gemm_streamk_status(&flags, 1));
        app::report(bad == 0 && flags == 0,
                    "mismatches=" + std::to_string(bad) + " status=" + std::to_string(flags));
    }
}

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(
        argc, argv, "rocwmma_streamk_gemm [M N K] [--blocks=B] [--verify]", {"--blocks="});
    uint32_t blocks = 0; // 0: one block per CU
    if(const char* v = o.value("--blocks=")) {
        char* end = nullptr;
        errno     = 0;
        const long long x = std::strtoll(v, &end, 10);
        if(!*v || *end || errno || x < 1 || x > 65536)
            app::usage_error(o, "--blocks= needs an integer in [1, 65536]");
        blocks = (uint32_t)x;
    }
    const auto d = app::sizes(o, {3});
    app::banner("W8A8 stream-K GEMM, int32 pieces summed in one launch (MI355X gfx950)");
    if(!d.empty()) {
        test_streamk(d[0], d[1], d[2], blocks, o.verify);
        return 0;
    }
    for(uint32_t s : {512u, 1024u, 2048u, 4096u}) test_streamk(s, s, 4096, blocks, o.verify);
    return 0;
}
