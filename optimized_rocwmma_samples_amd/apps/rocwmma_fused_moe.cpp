// rocwmma_fused_moe -- the MoE expert FFN on MI355X: routing, stable sort,
// per-expert SmoothQuant straight into expert-sorted rows, gate_up expert GEMM
// with SiLU(gate)*up in its epilogue (the sample's moe_gate_up_silu_kernel,
// rocwmma_fused_moe.cpp:96-158) and the requantization for the down GEMM,
// down expert GEMM, weighted combine.  The gate_up weights are interleaved
// once, before the timed launches (w8a8_moe_interleave_gate_up).
// Configurations and result line of the reference sample
// (rocwmma_fused_moe.cpp:227-245):
//   [FusedMoE] tokens=<T> hidden=<H> inter=<I> experts=<E> topk=<k>  <ms> ms  <TF> TFlops/s
// FLOPs = 2 * T * k * (2I * H + H * I): each routed row through both GEMMs
// (the sample counts K_gate_up for both GEMMs and assumes uniform routing, :163-165, :225).
// `rocwmma_fused_moe [tokens hidden inter experts topk]`.
#include "common.hpp"

static void test_fused_moe(uint32_t t, uint32_t h, uint32_t inter, uint32_t e, uint32_t k,
                           bool verify)
{
    const uint64_t seed = app::config_seed(5);
    auto           hx   = app::gen_activations(seed, t, h);
    auto           hl   = app::gen_normal(seed, app::kLogits, (size_t)t * e);
    auto           hs   = app::gen_uniform(seed, app::kExpertS, (size_t)e * h, 0.5, 2.0);
    auto           hwgu = app::gen_int8(seed, app::kB, (size_t)e * 2 * inter * h);
    auto           hsgu = app::gen_uniform(seed, app::kSb, (size_t)e * 2 * inter, 1e-3, 1e-2);
    auto           hwd  = app::gen_int8(seed, app::kWDown, (size_t)e * h * inter);
    auto           hsd  = app::gen_uniform(seed, app::kSbDown, (size_t)e * h, 1e-3, 1e-2);
    const uint32_t cap  = (uint32_t)w8a8_moe_sort_capacity(t, k, e, 32);
    app::Dev<uint16_t> dx(hx), y((size_t)cap * h), out((size_t)t * h);
    app::Dev<float>    dl(hl), ds(hs), dsgu(hsgu), dsd(hsd), w((size_t)t * k), ra(cap), r2(cap);
    app::Dev<float>    dsgu_il((size_t)e * 2 * inter);
    app::Dev<int8_t>   dwgu(hwgu), dwd(hwd), qa((size_t)cap * h), q2((size_t)cap * inter);
    app::Dev<int8_t>   dwgu_il((size_t)e * 2 * inter * h);
    CHECK_W8A8(w8a8_moe_interleave_gate_up(dwgu.p, dsgu.p, e, inter, h, h, dwgu_il.p, dsgu_il.p,
                                           nullptr));
    const size_t     fwsb = w8a8_moe_gate_up_silu_workspace_size(cap, inter);
    app::Dev<int8_t> fws(fwsb);
    app::Dev<int32_t>  ids((size_t)t * k), cnt(e), st(e + 1), pad(e), srt(cap), dst((size_t)t * k);
    const size_t       wsb = w8a8_moe_gemm_workspace_size(e, cap, h, inter);
    app::Dev<int8_t>   ws(wsb);
    const size_t       swsb = w8a8_moe_sort_workspace_size(t, k, e);
    app::Dev<int8_t>   sws(swsb);
    auto fn = [&] {
        CHECK_W8A8(w8a8_topk_softmax(dl.p, 0, w.p, ids.p, t, e, k, nullptr));
        CHECK_W8A8(w8a8_moe_sort(ids.p, t, k, e, 32, cnt.p, st.p, pad.p, srt.p, cap, dst.p,
                                 swsb ? sws.p : nullptr, swsb, nullptr));
        CHECK_W8A8(w8a8_moe_smoothquant(dx.p, ds.p, ids.p, qa.p, ra.p, t, h, k, e, 127.f, dst.p,
                                        cap, nullptr));
        CHECK_W8A8(w8a8_moe_gate_up_silu(e, cap, inter, h, qa.p, h, dwgu_il.p, ra.p, dsgu_il.p,
                                         1.f, 1.f, nullptr, st.p, cnt.p, q2.p, inter, r2.p, 127.f,
                                         fws.p, fwsb, nullptr));
        CHECK_W8A8(w8a8_moe_gemm(e, cap, h, inter, q2.p, inter, dwd.p, inter, (uint64_t)h * inter,
                                 y.p, h, r2.p, dsd.p, 1.f, 1.f, st.p, cnt.p, W8A8_OUT_F16,
                                 ws.p, wsb, nullptr));
        CHECK_W8A8(w8a8_moe_combine(y.p, h, cap, w.p, dst.p, t, k, h, out.p, h, nullptr));
    };
    const double ms    = app::bench_ms(fn, 3, 10);
    const double flops = 2.0 * t * k * (2.0 * inter * h + (double)h * inter);
    std::cout << "[FusedMoE] tokens=" << t << " hidden=" << h << " inter=" << inter
              << " experts=" << e << " topk=" << k << "  " << ms << " ms  "
              << flops / (ms * 1e-3) / 1e12 << " TFlops/s\n";
    if(verify) {
        // sampled rows of every expert, from the GPU's inputs: the gate_up
        // GEMM + SiLU*up + requant (q within one step of the CPU's, which
        // rounds the activation to fp16 before it quantizes, as the GPU does)
        // and the down GEMM (exact)
        const auto c = cnt.download(), s = st.download();
        const auto gqa = qa.download(), gq2 = q2.download();
        const auto gra = ra.download(), gr2 = r2.download();
        const auto gy = y.download();
        size_t     bad = 0, off = 0;
        for(uint32_t x = 0; x < e; ++x) {
            if(c[x] == 0) continue;
            std::vector<size_t> rows;
            for(size_t r : app::sample_rows(c[x], 8)) rows.push_back(s[x] + r);
            const auto a1 = app::cpu_gemm_i32(gqa.data(), hwgu.data() + (size_t)x * 2 * inter * h,
                                              cap, 2 * inter, h, rows);
            const auto a2 = app::cpu_gemm_i32(gq2.data(), hwd.data() + (size_t)x * h * inter, cap,
                                              h, inter, rows);
            for(size_t ri = 0; ri < rows.size(); ++ri) {
                std::vector<uint16_t> act(inter);
                const float*          sg = hsgu.data() + (size_t)x * 2 * inter;
                for(uint32_t j = 0; j < inter; ++j) {
                    const float g = app::h2f(app::cpu_dequant(a1[ri * 2 * inter + j], gra[rows[ri]], sg[j]));
                    const float u = app::h2f(app::cpu_dequant(a1[ri * 2 * inter + inter + j],
                                                              gra[rows[ri]], sg[inter + j]));
                    act[j] = app::f2h(g / (1.f + std::exp(-g)) * u);
                }
                const std::vector<float> ones(inter, 1.f);
                std::vector<int8_t>      qc(inter);
                float                    rc = 0.f;
                app::cpu_smoothquant(act.data(), ones.data(), qc.data(), &rc, 1, inter, 127.f);
                for(uint32_t j = 0; j < inter; ++j) {
                    const int d = std::abs((int)gq2[rows[ri] * inter + j] - (int)qc[j]);
                    bad += d > 1;
                    off += d == 1;
                }
                bad += std::fabs(gr2[rows[ri]] - rc) > 1e-3f * rc;
                for(uint32_t j = 0; j < h; ++j)
                    bad += gy[rows[ri] * h + j]
                           != app::cpu_dequant(a2[ri * h + j], gr2[rows[ri]], hsd[(size_t)x * h + j]);
            }
        }
        app::report(bad == 0, "mismatches on sampled rows=" + std::to_string(bad)
                                  + " (q one step apart: " + std::to_string(off) + ")");
    }
}

int main(int argc, char* argv[])
{
    const app::Options o = app::parse(
        argc, argv, "rocwmma_fused_moe [TOKENS HIDDEN INTER EXPERTS TOPK] [--verify]");
    const auto d = app::sizes(o, {5});
    if(!d.empty() && d[4] > d[3]) app::usage_error(o, "TOPK must not exceed EXPERTS");
    app::banner("W8A8 MoE FFN (MI355X gfx950)");
    if(!d.empty()) {
        test_fused_moe(d[0], d[1], d[2], d[3], d[4], o.verify);
        return 0;
    }
    test_fused_moe(3328, 4096, 14336, 8, 2, o.verify);
    test_fused_moe(3328, 4096, 14336, 32, 5, o.verify);
    test_fused_moe(3328, 7168, 2048, 64, 6, o.verify);
    test_fused_moe(4096, 4096, 14336, 8, 2, o.verify);
    return 0;
}
