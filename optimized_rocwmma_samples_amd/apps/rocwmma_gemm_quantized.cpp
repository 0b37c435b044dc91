// rocwmma_gemm_quantized -- W8A8 int8 GEMM with fused dequant on MI355X.
// Replaces the FP8 tensor-scale sample (rocwmma_gemm_quantized.cpp:197-268):
// `rocwmma_gemm_quantized [M N K] [--sample-layout]`, default sizes 3840x4096x4096,
// 4096^3, 8192^3, result line
//   [QuantGEMM-INT8] M=<M> N=<N> K=<K>  <ms> ms  <TF> TFlops/s (<mode>)
// Default mode: A [M,K] row-major, W [N,K], per-token x per-channel fp32 scales
// (the W8A8 layout).  --sample-layout: the sample's A col-major / B [K,N] with
// tensor scales 1/127 (:205, :226).  Any M, N, K is accepted (the sample skips
// sizes that are not tile multiples, :199-203).
#include "common.hpp"

static void test_quant_gemm(uint32_t m, uint32_t n, uint32_t k, bool sample, bool verify)
{
    const uint64_t seed = app::config_seed(2);
    auto           ha   = app::gen_int8(seed, app::kA, (size_t)m * k); // [m,k], or [k,m] for the sample layout
    auto           hb   = app::gen_int8(seed, app::kB, (size_t)n * k); // [n,k], or [k,n]
    auto           hsa  = app::gen_uniform(seed, app::kSa, m, 1e-3, 1e-2);
    auto           hsb  = app::gen_uniform(seed, app::kSb, n, 1e-3, 1e-2);
    app::Dev<int8_t>   da(ha), db(hb);
    app::Dev<float>    dsa(hsa), dsb(hsb);
    app::Dev<uint16_t> dc((size_t)m * n);
    const int    layout = sample ? W8A8_LAYOUT_A_COL_B_KN : W8A8_LAYOUT_A_ROW_B_NK;
    const size_t wsb    = w8a8_gemm_workspace_size(m, n, k, layout);
    app::Dev<int8_t> ws(wsb);
    const uint32_t lda = sample ? m : k, ldb = sample ? n : k;
    const float*   sa  = sample ? nullptr : dsa.p;
    const float*   sb  = sample ? nullptr : dsb.p;
    const float    ts  = sample ? 1.f / 127.f : 1.f;
    auto fn = [&](void* c, int out) {
        CHECK_W8A8(w8a8_gemm(m, n, k, da.p, db.p, c, lda, ldb, n, sa, sb, ts, ts, out, layout,
                             wsb ? ws.p : nullptr, wsb, nullptr));
    };
    const double ms = app::bench_ms([&] { fn(dc.p, W8A8_OUT_F16); });
    const double tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12;
    std::cout << "[QuantGEMM-INT8] M=" << m << " N=" << n << " K=" << k << "  " << ms << " ms  "
              << tf << " TFlops/s ("
              << (sample ? "sample layout, tensor scales" : "per-token x per-channel dequant")
              << ")\n";
    if(verify) {
        app::Dev<int32_t> di((size_t)m * n);
        fn(di.p, W8A8_OUT_I32);
        const auto gi = di.download();
        const auto gc = dc.download();
        // row-major A [m,k] and B [n,k] copies for the CPU check
        std::vector<int8_t> a = ha, b = hb;
        if(sample) {
            for(size_t i = 0; i < m; ++i)
                for(size_t h = 0; h < k; ++h) a[i * k + h] = ha[h * m + i];
            for(size_t j = 0; j < n; ++j)
                for(size_t h = 0; h < k; ++h) b[j * k + h] = hb[h * n + j];
        }
        const auto rows = app::sample_rows(m, 256);
        const auto acc  = app::cpu_gemm_i32(a.data(), b.data(), m, n, k, rows);
        size_t     bad_i = 0, bad_f = 0;
        for(size_t ri = 0; ri < rows.size(); ++ri)
            for(size_t j = 0; j < n; ++j) {
                const int32_t v = acc[ri * n + j];
                bad_i += gi[rows[ri] * n + j] != v;
                const uint16_t e = sample ? app::f2h((float)v * (ts * ts))
                                          : app::cpu_dequant(v, hsa[rows[ri]], hsb[j]);
                bad_f += gc[rows[ri] * n + j] != e;
            }
        app::report(bad_i == 0 && bad_f == 0,
                    std::to_string(rows.size()) + " rows: int32 mismatches=" +
                        std::to_string(bad_i) + " fp16 mismatches=" + std::to_string(bad_f));
    }
}

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(
        argc, argv, "rocwmma_gemm_quantized [M N K] [--sample-layout] [--verify]",
        {"--sample-layout"});
    const bool sample = o.has("--sample-layout");
    const auto d      = app::sizes(o, {3});
    app::banner("W8A8 Quantized GEMM, int8 MFMA (MI355X gfx950)");
    if(!d.empty()) {
        test_quant_gemm(d[0], d[1], d[2], sample, o.verify);
        return 0;
    }
    test_quant_gemm(3840, 4096, 4096, sample, o.verify);
    test_quant_gemm(4096, 4096, 4096, sample, o.verify);
    test_quant_gemm(8192, 8192, 8192, sample, o.verify);
    return 0;
}
