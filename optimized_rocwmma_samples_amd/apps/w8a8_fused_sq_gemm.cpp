// w8a8_fused_sq_gemm -- SmoothQuant + W8A8 GEMM for one linear layer (BASELINE
// config 3: Llama-3-8B projections at M in {512, 2048, 8192}).
// `w8a8_fused_sq_gemm [M N K]`; result line
//   [FusedSQ-GEMM] M=<M> N=<N> K=<K>  <ms> ms  <TF> TFlops/s
// timing both kernels (quantizer + GEMM) per layer.
#include "common.hpp"

static void test_fused(uint32_t m, uint32_t n, uint32_t k, bool verify)
{
    const uint64_t seed = app::config_seed(3);
    auto           hx   = app::gen_activations(seed, m, k);
    auto           hs   = app::gen_uniform(seed, app::kS, k, 0.5, 2.0);
    auto           hw   = app::gen_int8(seed, app::kB, (size_t)n * k);
    auto           hsb  = app::gen_uniform(seed, app::kSb, n, 1e-3, 1e-2);
    app::Dev<uint16_t> dx(hx), dc((size_t)m * n);
    app::Dev<float>    ds(hs), dsb(hsb), dr(m);
    app::Dev<int8_t>   dw(hw), dq((size_t)m * k);
    const size_t       wsb = w8a8_gemm_workspace_size(m, n, k, W8A8_LAYOUT_A_ROW_B_NK);
    app::Dev<int8_t>   ws(wsb);
    auto fn = [&] {
        CHECK_W8A8(w8a8_fused_sq_gemm(dx.p, ds.p, dw.p, dsb.p, dc.p, m, n, k, 0, 0, 0, dq.p, dr.p,
                                      ws.p, wsb, nullptr));
    };
    const double ms = app::bench_ms(fn);
    std::cout << "[FusedSQ-GEMM] M=" << m << " N=" << n << " K=" << k << "  " << ms << " ms  "
              << 2.0 * m * n * k / (ms * 1e-3) / 1e12 << " TFlops/s\n";
    if(verify) {
        std::vector<int8_t> q((size_t)m * k);
        std::vector<float>  r(m);
        app::cpu_smoothquant(hx.data(), hs.data(), q.data(), r.data(), m, k, 127.f);
        const auto rows = app::sample_rows(m, 128);
        const auto acc  = app::cpu_gemm_i32(q.data(), hw.data(), m, n, k, rows);
        const auto gq = dq.download();
        const auto gc = dc.download();
        size_t     bad_q = 0, bad_c = 0;
        for(size_t i = 0; i < q.size(); ++i) bad_q += gq[i] != q[i];
        for(size_t ri = 0; ri < rows.size(); ++ri)
            for(size_t j = 0; j < n; ++j)
                bad_c += gc[rows[ri] * n + j] != app::cpu_dequant(acc[ri * n + j], r[rows[ri]], hsb[j]);
        app::report(bad_q == 0 && bad_c == 0, "q mismatches=" + std::to_string(bad_q) +
                                                  ", fp16 mismatches on " +
                                                  std::to_string(rows.size()) +
                                                  " rows=" + std::to_string(bad_c));
    }
}

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(argc, argv, "w8a8_fused_sq_gemm [M N K] [--verify]");
    const auto         d = app::sizes(o, {3});
    app::banner("W8A8 fused SmoothQuant + GEMM (MI355X gfx950)");
    if(!d.empty()) {
        test_fused(d[0], d[1], d[2], o.verify);
        return 0;
    }
    const uint32_t shapes[4][2] = {{4096, 6144}, {4096, 4096}, {4096, 28672}, {14336, 4096}};
    for(uint32_t m : {512u, 2048u, 8192u})
        for(auto& s : shapes) test_fused(m, s[1], s[0], o.verify);
    return 0;
}
