// rocwmma_grouped_gemm -- grouped W8A8 GEMM (one launch for many problems).
// Group lists and result lines of the reference sample
// (rocwmma_grouped_gemm.cpp:236-268):
//   [GroupedGEMM] G=<G>  (MxNxK) (MxNxK) ...
//     total <ms> ms  <TF> TFlops/s
#include "common.hpp"

#include <array>

static void test_grouped(const std::vector<std::array<uint32_t, 3>>& sizes, bool verify)
{
    const uint64_t seed = app::config_seed(5);
    const size_t   G    = sizes.size();
    std::vector<std::vector<int8_t>>   ha(G), hb(G);
    std::vector<std::vector<float>>    hsa(G), hsb(G);
    std::vector<std::unique_ptr<app::Dev<int8_t>>>   da, db;
    std::vector<std::unique_ptr<app::Dev<float>>>    dsa, dsb;
    std::vector<std::unique_ptr<app::Dev<uint16_t>>> dc;
    std::vector<w8a8_group_desc> desc(G);
    double                       flops = 0;
    for(size_t g = 0; g < G; ++g) {
        const auto [m, n, k] = sizes[g];
        ha[g]  = app::gen_int8(seed + g, app::kA, (size_t)m * k);
        hb[g]  = app::gen_int8(seed + g, app::kB, (size_t)n * k);
        hsa[g] = app::gen_uniform(seed + g, app::kSa, m, 1e-3, 1e-2);
        hsb[g] = app::gen_uniform(seed + g, app::kSb, n, 1e-3, 1e-2);
        da.emplace_back(new app::Dev<int8_t>(ha[g]));
        db.emplace_back(new app::Dev<int8_t>(hb[g]));
        dsa.emplace_back(new app::Dev<float>(hsa[g]));
        dsb.emplace_back(new app::Dev<float>(hsb[g]));
        dc.emplace_back(new app::Dev<uint16_t>((size_t)m * n));
        desc[g] = w8a8_group_desc{da[g]->p, db[g]->p, dc[g]->p, dsa[g]->p, dsb[g]->p, m, n, k,
                                  k,        k,        n,        1.f,       1.f};
        flops += 2.0 * m * n * k;
    }
    const size_t     wsb = w8a8_grouped_gemm_workspace_size((uint32_t)G);
    app::Dev<int8_t> ws(wsb);
    auto fn = [&] {
        CHECK_W8A8(w8a8_grouped_gemm(desc.data(), (uint32_t)G, W8A8_OUT_F16, ws.p, wsb, nullptr));
    };
    const double ms = app::bench_ms(fn);
    std::cout << "[GroupedGEMM] G=" << G << "  ";
    for(auto& s : sizes) std::cout << "(" << s[0] << "x" << s[1] << "x" << s[2] << ") ";
    std::cout << "\n  total " << ms << " ms  " << flops / (ms * 1e-3) / 1e12 << " TFlops/s\n";
    if(verify) {
        size_t bad = 0, rows_checked = 0;
        for(size_t g = 0; g < G; ++g) {
            const auto [m, n, k] = sizes[g];
            const auto rows      = app::sample_rows(m, 64);
            const auto acc = app::cpu_gemm_i32(ha[g].data(), hb[g].data(), m, n, k, rows);
            const auto gc  = dc[g]->download();
            for(size_t ri = 0; ri < rows.size(); ++ri)
                for(size_t j = 0; j < n; ++j)
                    bad += gc[rows[ri] * n + j]
                           != app::cpu_dequant(acc[ri * n + j], hsa[g][rows[ri]], hsb[g][j]);
            rows_checked += rows.size();
        }
        app::report(bad == 0, std::to_string(rows_checked) + " rows, mismatches=" +
                                  std::to_string(bad));
    }
}

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(argc, argv, "rocwmma_grouped_gemm [--verify]");
    (void)app::sizes(o, {});
    app::banner("W8A8 Grouped GEMM (MI355X gfx950)");
    test_grouped({{256, 4096, 4096}, {512, 4096, 4096}, {128, 4096, 4096}, {768, 4096, 4096}},
                 o.verify);
    test_grouped({{1024, 4096, 4096}, {1024, 4096, 4096}, {1024, 4096, 4096}, {1024, 4096, 4096}},
                 o.verify);
    test_grouped({{512, 1024, 2048}, {512, 2048, 2048}, {512, 4096, 2048}}, o.verify);
    return 0;
}
