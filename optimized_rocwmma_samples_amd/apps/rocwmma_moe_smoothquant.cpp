// rocwmma_moe_smoothquant -- per-expert SmoothQuant on MI355X.
// Configurations and result line of the reference sample
// (rocwmma_moe_smoothquant.cpp:188-204):
//   [MoE-SmoothQuant] tokens=<T> hidden=<H> experts=<E> topk=<k>  <ms> ms  <GB/s> GB/s
// bytes = 2TH + 4EH + 4Tk + TkH + 4Tk (:186-187).  Expert ids: k distinct per
// token from std::mt19937(42), as the sample draws them (:149-163).
#include "common.hpp"

#include <random>
#include <set>

static void test_moe_smoothquant(uint32_t tokens, uint32_t hidden, uint32_t experts,
                                 uint32_t topk, bool verify)
{
    std::mt19937                       rng(42);
    std::uniform_int_distribution<int> edist(0, (int)experts - 1);
    std::vector<int32_t>               hids((size_t)tokens * topk);
    for(uint32_t t = 0; t < tokens; ++t) {
        std::set<int> used;
        for(uint32_t k = 0; k < topk; ++k) {
            int e = edist(rng);
            while(used.count(e)) e = edist(rng);
            used.insert(e);
            hids[(size_t)t * topk + k] = e;
        }
    }
    const uint64_t seed = app::config_seed(5);
    auto           hx   = app::gen_activations(seed, tokens, hidden);
    auto           hs   = app::gen_uniform(seed, app::kExpertS, (size_t)experts * hidden, 0.5, 2.0);
    const size_t   rows = (size_t)tokens * topk;
    app::Dev<uint16_t> dx(hx);
    app::Dev<float>    ds(hs);
    app::Dev<int32_t>  did(hids);
    app::Dev<int8_t>   dq(rows * hidden);
    app::Dev<float>    dr(rows);
    auto fn = [&] {
        CHECK_W8A8(w8a8_moe_smoothquant(dx.p, ds.p, did.p, dq.p, dr.p, tokens, hidden, topk,
                                        experts, 127.f, nullptr, 0, nullptr));
    };
    const double ms = app::bench_ms(fn);
    const double bytes = 2.0 * tokens * hidden + 4.0 * experts * hidden + 4.0 * tokens * topk
                         + (double)rows * hidden + 4.0 * rows;
    std::cout << "[MoE-SmoothQuant] tokens=" << tokens << " hidden=" << hidden
              << " experts=" << experts << " topk=" << topk << "  " << ms << " ms  "
              << bytes / (ms * 1e-3) / 1e9 << " GB/s\n";
    if(verify) {
        const auto gq = dq.download();
        const auto gr = dr.download();
        size_t     bad = 0;
        std::vector<int8_t> q(hidden);
        float               r;
        for(size_t p = 0; p < rows; ++p) {
            const int e = hids[p];
            app::cpu_smoothquant(hx.data() + (p / topk) * hidden, hs.data() + (size_t)e * hidden,
                                 q.data(), &r, 1, hidden, 127.f);
            for(uint32_t j = 0; j < hidden; ++j) bad += gq[p * hidden + j] != q[j];
            bad += std::memcmp(&gr[p], &r, 4) != 0;
        }
        app::report(bad == 0, "mismatches=" + std::to_string(bad));
    }
}

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(argc, argv, "rocwmma_moe_smoothquant [--verify]");
    (void)app::sizes(o, {});
    app::banner("W8A8 MoE SmoothQuant (MI355X gfx950)");
    test_moe_smoothquant(3328, 4096, 32, 5, o.verify);
    test_moe_smoothquant(3328, 4096, 8, 2, o.verify);
    test_moe_smoothquant(3328, 8192, 64, 5, o.verify);
    return 0;
}
