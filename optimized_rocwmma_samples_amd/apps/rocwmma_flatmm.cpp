// rocwmma_flatmm -- W8A8 GEMM over pre-shuffled ("packed") weights on MI355X.
// The reference's FlatMM sample describes weights pre-shuffled into MFMA
// register order and streamed past LDS (rocwmma_flatmm.cpp:12-16) and keeps
// them row-major; here w8a8_pack_weights produces that layout once and
// w8a8_gemm_packed streams it (1 KiB contiguous per wave-load).
// `rocwmma_flatmm [M N K]`; default: the sample's shapes (M in 128..4096,
// N = K = 4096, :203-207) and config 4's decode shapes.  Result line
//   [FlatMM] M=<M> N=<N> K=<K>  packed weights  <ms> ms  <TF> TFlops/s  <GB/s> GB/s
#include "common.hpp"

static void test_flatmm(uint32_t m, uint32_t n, uint32_t k, bool verify)
{
    const uint64_t seed = app::config_seed(4);
    auto           ha   = app::gen_int8(seed, app::kA, (size_t)m * k);
    auto           hw   = app::gen_int8(seed, app::kB, (size_t)n * k);
    auto           hsa  = app::gen_uniform(seed, app::kSa, m, 1e-3, 1e-2);
    auto           hsb  = app::gen_uniform(seed, app::kSb, n, 1e-3, 1e-2);
    app::Dev<int8_t>   da(ha), dw(hw);
    app::Dev<float>    dsa(hsa), dsb(hsb);
    app::Dev<uint16_t> dc((size_t)m * n);
    const size_t       pbytes = w8a8_pack_weights_size(n, k);
    app::Dev<int8_t>   dp(pbytes);
    CHECK_W8A8(w8a8_pack_weights(dw.p, n, k, k, dp.p, pbytes, nullptr));
    // split-K workspace for 32 < M <= 64 (caller-allocated, as the reference's
    // split-K sample allocates its own, rocwmma_gemm_splitk.cpp:214)
    const size_t     wsb = w8a8_gemm_packed_workspace_size(m, n, k);
    app::Dev<int8_t> dws(wsb > 0 ? wsb : 16);
    auto fn = [&](void* c, int out) {
        CHECK_W8A8(w8a8_gemm_packed(m, n, k, da.p, dp.p, c, k, n, dsa.p, dsb.p, 1.f, 1.f, out,
                                    wsb > 0 ? dws.p : nullptr, wsb, nullptr));
    };
    const double ms    = app::bench_ms([&] { fn(dc.p, W8A8_OUT_F16); });
    const double bytes = (double)n * k + (double)m * k + 4.0 * (m + n) + 2.0 * m * n;
    std::cout << "[FlatMM] M=" << m << " N=" << n << " K=" << k << "  packed weights  " << ms
              << " ms  " << 2.0 * m * n * k / (ms * 1e-3) / 1e12 << " TFlops/s  "
              << bytes / (ms * 1e-3) / 1e9 << " GB/s\n";
    if(verify) {
        app::Dev<int32_t> di((size_t)m * n);
        fn(di.p, W8A8_OUT_I32);
        const auto rows = app::sample_rows(m, 64);
        const auto acc  = app::cpu_gemm_i32(ha.data(), hw.data(), m, n, k, rows);
        const auto gi = di.download();
        const auto gc = dc.download();
        size_t     bad = 0;
        for(size_t ri = 0; ri < rows.size(); ++ri)
            for(size_t j = 0; j < n; ++j) {
                bad += gi[rows[ri] * n + j] != acc[ri * n + j];
                bad += gc[rows[ri] * n + j] != app::cpu_dequant(acc[ri * n + j], hsa[rows[ri]], hsb[j]);
            }
        app::report(bad == 0, "mismatches=" + std::to_string(bad));
    }
}

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(argc, argv, "rocwmma_flatmm [M N K] [--verify]");
    const auto         d = app::sizes(o, {3});
    app::banner("W8A8 GEMM over packed weights (MI355X gfx950)");
    if(!d.empty()) {
        test_flatmm(d[0], d[1], d[2], o.verify);
        return 0;
    }
    for(uint32_t m : {128u, 256u, 512u, 1024u, 4096u}) test_flatmm(m, 4096, 4096, o.verify);
    for(uint32_t m : {1u, 16u, 64u}) {
        test_flatmm(m, 28672, 8192, o.verify);
        test_flatmm(m, 8192, 28672, o.verify);
    }
    return 0;
}
