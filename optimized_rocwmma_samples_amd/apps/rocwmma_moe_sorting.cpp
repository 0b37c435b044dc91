// rocwmma_moe_sorting -- deterministic MoE token sort on MI355X.
// Command line and result line of the reference sample
// (rocwmma_moe_sorting.cpp:189-209): `rocwmma_moe_sorting [tokens experts topk]`,
// default 3328 x 8 x 4 (unit 32), then (E, k) in (16,2) (32,4) (64,5) (128,8);
//   [MoE Sorting] tokens=<T> experts=<E> topk=<k> unit=<u>  <ms> ms  <GB/s> GB/s
// with the sample's bytes formula (8Tk + 4 * padded bound, :186-188).
#include "common.hpp"

#include <random>

static void test_sort(uint32_t tokens, uint32_t experts, uint32_t topk, uint32_t unit, bool verify)
{
    const uint32_t       total = tokens * topk;
    std::vector<int32_t> ids(total);
    for(uint32_t t = 0; t < tokens; ++t) { // k distinct experts per token
        std::vector<int32_t> ex(experts);
        for(uint32_t e = 0; e < experts; ++e) ex[e] = (int32_t)e;
        std::shuffle(ex.begin(), ex.end(), std::default_random_engine(t));
        for(uint32_t k = 0; k < topk; ++k) ids[(size_t)t * topk + k] = ex[k];
    }
    const uint32_t    cap = (uint32_t)w8a8_moe_sort_capacity(tokens, topk, experts, unit);
    app::Dev<int32_t> did(ids), cnt(experts), st(experts + 1), pad(experts), srt(cap), dst(total);
    const size_t      wsb = w8a8_moe_sort_workspace_size(tokens, topk, experts);
    app::Dev<int8_t>  ws(wsb);
    auto fn = [&] {
        CHECK_W8A8(w8a8_moe_sort(did.p, tokens, topk, experts, unit, cnt.p, st.p, pad.p, srt.p,
                                 cap, dst.p, wsb ? ws.p : nullptr, wsb, nullptr));
    };
    const double ms = app::bench_ms(fn, 3, 10);
    std::cout << "[MoE Sorting] tokens=" << tokens << " experts=" << experts << " topk=" << topk
              << " unit=" << unit << "  " << ms << " ms  "
              << (8.0 * total + 4.0 * cap) / (ms * 1e-3) / 1e9 << " GB/s\n";
    if(verify) { // stable counting sort on the host
        std::vector<int32_t> c(experts, 0), s(experts + 1, 0);
        for(int32_t e : ids) c[e]++;
        for(uint32_t e = 0; e < experts; ++e) s[e + 1] = s[e] + (c[e] + unit - 1) / unit * unit;
        std::vector<int32_t> sorted(cap, -1), cur(experts, 0), d(total);
        for(uint32_t p = 0; p < total; ++p) {
            const int32_t slot = s[ids[p]] + cur[ids[p]]++;
            sorted[slot]       = (int32_t)(p / topk);
            d[p]               = slot;
        }
        const bool ok = cnt.download() == c && st.download() == s && srt.download() == sorted
                        && dst.download() == d;
        app::report(ok, "count/start/sorted ids/destination rows");
    }
}

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(argc, argv, "rocwmma_moe_sorting [TOKENS EXPERTS TOPK] [--verify]");
    const auto         d = app::sizes(o, {3});
    uint32_t           tokens = 3328, experts = 8, topk = 4, unit = 32;
    if(!d.empty()) {
        tokens  = d[0];
        experts = d[1];
        topk    = d[2];
        if(topk > experts) app::usage_error(o, "TOPK must not exceed EXPERTS");
    }
    app::banner("W8A8 MoE Sorting, stable (MI355X gfx950)");
    test_sort(tokens, experts, topk, unit, o.verify);
    const uint32_t cfg[4][2] = {{16, 2}, {32, 4}, {64, 5}, {128, 8}};
    for(auto& c : cfg)
        if(c[1] <= c[0]) test_sort(tokens, c[0], c[1], unit, o.verify);
    return 0;
}
