// rocwmma_gemm_splitk -- decode-shaped (skinny) W8A8 GEMM on MI355X.
// Stands in for the reference's split-K and stream-K samples
// (rocwmma_gemm_splitk.cpp:251-263, rocwmma_streamk_gemm.cpp:286-297): m <= 64
// runs the weight-streaming kernel that splits K across the waves of each
// block (int32 partials summed in LDS, one launch, no workspace), or 64 x 128
// tiles where those stream the row-major weights faster; tiles that fill at
// most half of the CUs are split along K across blocks into the caller's
// workspace (int32 partials, a fixup launch sums them), like the reference's
// workspace-based split-K (:214).
// `rocwmma_gemm_splitk [M N K]`; default: BASELINE config 4, the Llama-70B MLP
// weights [28672, 8192] and [8192, 28672] at M in {1, 16, 64}, then the
// reference's shapes.  Result line
//   [SplitK-GEMM] M=<M> N=<N> K=<K> split_k=<in-block|workspace|none>  <ms> ms  <TF> TFlops/s  <GB/s> GB/s
// (GB/s = weights + activations + scales + output once).
#include "common.hpp"

static void test_decode(uint32_t m, uint32_t n, uint32_t k, bool verify)
{
    const uint64_t seed = app::config_seed(4);
    auto           ha   = app::gen_int8(seed, app::kA, (size_t)m * k);
    auto           hw   = app::gen_int8(seed, app::kB, (size_t)n * k);
    auto           hsa  = app::gen_uniform(seed, app::kSa, m, 1e-3, 1e-2);
    auto           hsb  = app::gen_uniform(seed, app::kSb, n, 1e-3, 1e-2);
    app::Dev<int8_t>   da(ha), dw(hw);
    app::Dev<float>    dsa(hsa), dsb(hsb);
    app::Dev<uint16_t> dc((size_t)m * n);
    const size_t       wsb = w8a8_gemm_workspace_size(m, n, k, W8A8_LAYOUT_A_ROW_B_NK);
    app::Dev<int8_t>   ws(wsb);
    auto fn = [&](void* c, int out) {
        CHECK_W8A8(w8a8_gemm(m, n, k, da.p, dw.p, c, k, k, n, dsa.p, dsb.p, 1.f, 1.f, out,
                             W8A8_LAYOUT_A_ROW_B_NK, wsb ? ws.p : nullptr, wsb, nullptr));
    };
    const double ms    = app::bench_ms([&] { fn(dc.p, W8A8_OUT_F16); });
    const double bytes = (double)n * k + (double)m * k + 4.0 * (m + n) + 2.0 * m * n;
    std::cout << "[SplitK-GEMM] M=" << m << " N=" << n << " K=" << k
              << " split_k=" << (wsb ? "workspace" : m <= 64 ? "in-block" : "none") << "  " << ms
              << " ms  "
              << 2.0 * m * n * k / (ms * 1e-3) / 1e12 << " TFlops/s  "
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
    const app::Options o = app::parse(argc, argv, "rocwmma_gemm_splitk [M N K] [--verify]");
    const auto         d = app::sizes(o, {3});
    app::banner("W8A8 decode GEMM, split-K inside the block (MI355X gfx950)");
    if(!d.empty()) {
        test_decode(d[0], d[1], d[2], o.verify);
        return 0;
    }
    for(uint32_t m : {1u, 16u, 64u}) {
        test_decode(m, 28672, 8192, o.verify);
        test_decode(m, 8192, 28672, o.verify);
    }
    test_decode(512, 512, 16384, o.verify);
    test_decode(1024, 1024, 16384, o.verify);
    test_decode(2048, 2048, 8192, o.verify);
    test_decode(4096, 4096, 4096, o.verify);
    return 0;
}
