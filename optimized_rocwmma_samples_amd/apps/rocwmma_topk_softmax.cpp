// rocwmma_topk_softmax -- softmax + top-k routing on MI355X.
// Command line and result line of the reference sample
// (rocwmma_topk_softmax.cpp:237-257): `rocwmma_topk_softmax [tokens experts topk]`,
// default 128 x 8 x 4, then 3328 tokens with (E, k) in (8,2) (16,2) (32,5) (64,5);
//   [TopK-Softmax] tokens=<T> experts=<E> topk=<k>  <ms> ms  <GB/s> GB/s
// fp16 logits as in the sample (:42); bytes = 2TE + 8Tk.
#include "common.hpp"

static void test_topk(uint32_t t, uint32_t e, uint32_t k, bool verify)
{
    auto                  lf = app::gen_normal(app::config_seed(5), app::kLogits, (size_t)t * e);
    std::vector<uint16_t> hl(lf.size());
    for(size_t i = 0; i < lf.size(); ++i) hl[i] = app::f2h(lf[i]);
    app::Dev<uint16_t> dl(hl);
    app::Dev<float>    dw((size_t)t * k);
    app::Dev<int32_t>  di((size_t)t * k);
    auto fn = [&] { CHECK_W8A8(w8a8_topk_softmax(dl.p, 1, dw.p, di.p, t, e, k, nullptr)); };
    const double ms = app::bench_ms(fn);
    std::cout << "[TopK-Softmax] tokens=" << t << " experts=" << e << " topk=" << k << "  " << ms
              << " ms  " << (2.0 * t * e + 8.0 * t * k) / (ms * 1e-3) / 1e9 << " GB/s\n";
    if(verify) { // ids: highest logits first, lower id on ties
        const auto gi  = di.download();
        size_t     bad = 0;
        for(uint32_t r = 0; r < t; ++r) {
            std::vector<int> order(e);
            for(uint32_t x = 0; x < e; ++x) order[x] = (int)x;
            std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
                return app::h2f(hl[(size_t)r * e + a]) > app::h2f(hl[(size_t)r * e + b]);
            });
            for(uint32_t x = 0; x < k; ++x) bad += gi[(size_t)r * k + x] != order[x];
        }
        app::report(bad == 0, "id mismatches=" + std::to_string(bad));
    }
}

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(argc, argv, "rocwmma_topk_softmax [TOKENS EXPERTS TOPK] [--verify]");
    const auto         d = app::sizes(o, {3});
    uint32_t           t = 128, e = 8, k = 4;
    if(!d.empty()) {
        t = d[0];
        e = d[1];
        k = d[2];
        if(k > e) app::usage_error(o, "TOPK must not exceed EXPERTS");
    }
    app::banner("W8A8 MoE TopK-Softmax (MI355X gfx950)");
    test_topk(t, e, k, o.verify);
    const uint32_t cfg[4][2] = {{8, 2}, {16, 2}, {32, 5}, {64, 5}};
    for(auto& c : cfg) test_topk(3328, c[0], c[1], o.verify);
    return 0;
}
