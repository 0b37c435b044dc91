// Host check of the MoE tile schedule (MoeShape, tail_split and xcd_remap as
// the MoE kernels use them, gemm_i8_grouped_kernel.hpp), compiled and run by
// test_moe_plan_cpu.py.
//
// For random expert row counts (empty experts, rests of a few rows, whole
// tile rows, rests just above and below the wide tile's height), column
// counts, k-tile counts and CU counts, with and without the tail split, it
// walks every block of the launch the way the kernel does and checks by brute
// force that:
//   * every logical tile is run by exactly one block (whole tiles) or by
//     exactly `parts` blocks, one per k-piece (split tiles), and each XCD's
//     whole-tile blocks take a contiguous, increasing range of tiles;
//   * the tiles of every expert, C tiles then W tiles (MoeShape::origin),
//     cover each of its (row, column) outputs exactly once, and no tile
//     starts past its expert's rows or the columns.
// Logical ids are mapped to experts through the per-expert tile counts (the
// prefix sums find_slot forms on the GPU).  Prints "OK <cases>" on success,
// the first failure otherwise (status 1).
#include "../optimized_rocwmma_samples_amd/csrc/gemm_i8_grouped_kernel.hpp"

#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

using namespace w8a8::gemm;

template <class C, class W>
static int check(const std::vector<uint32_t>& rows, uint32_t n, uint32_t nk, uint32_t cus,
                 bool split, long case_id)
{
    using S        = MoeShape<C, W>;
    const size_t E = rows.size();
    uint32_t     total = 0, wide_tiles = 0;
    for(size_t e = 0; e < E; ++e) {
        total += S::tiles(rows[e], n);
        wide_tiles += S::w_tiles(rows[e], n);
    }
    const TailSplit sp = tail_split(total, cus, nk, split);
    auto fail = [&](const char* what, long a, long b) {
        std::printf("FAIL case %ld (experts %zu n %u nk %u cus %u split %d tiles %u wide %u): "
                    "%s (%ld, %ld)\n", case_id, E, n, nk, cus, (int)split, total, wide_tiles,
                    what, a, b);
        return 1;
    };
    if(sp.base + sp.left != total) return fail("base + left", sp.base, total);
    if(sp.left * sp.parts > (cus > 0 ? cus : 1)) return fail("split blocks > CUs", sp.left, sp.parts);

    std::vector<int>  use(total, 0);
    std::vector<long> last(8, -1);
    for(uint32_t b = 0; b < sp.base; ++b) {
        const uint32_t lid = xcd_remap(b, sp.base);
        if(lid >= sp.base) return fail("whole tile id out of range", b, lid);
        if(last[b % 8] >= 0 && (long)lid != last[b % 8] + 1)
            return fail("tiles of an XCD not contiguous", b, lid);
        last[b % 8] = lid;
        ++use[lid];
    }
    for(uint32_t x = 0; x < sp.left * sp.parts; ++x) ++use[sp.base + x / sp.parts];
    for(uint32_t l = 0; l < total; ++l)
        if(use[l] != (l < sp.base ? 1 : (int)sp.parts)) return fail("tile run count", l, use[l]);

    // coverage of every expert's outputs, 1 cell per (row, column)
    for(size_t e = 0; e < E; ++e) {
        if(rows[e] == 0) {
            if(S::tiles(0, n) != 0) return fail("tiles of an empty expert", (long)e, 0);
            continue;
        }
        std::vector<uint8_t> cov((size_t)rows[e] * n, 0);
        const uint32_t       nt = S::tiles(rows[e], n);
        for(uint32_t j = 0; j < nt; ++j) {
            uint32_t m0, n0;
            bool     wide;
            S::origin(j, rows[e], n, m0, n0, wide);
            if(wide != (j >= S::c_tiles(rows[e], n))) return fail("shape of a tile", (long)e, j);
            if(m0 >= rows[e] || n0 >= n) return fail("tile outside its expert", (long)e, j);
            const uint32_t bm = wide ? W::kBM : C::kBM, bn = wide ? W::kBN : C::kBN;
            for(uint32_t r = m0; r < std::min(m0 + bm, rows[e]); ++r)
                for(uint32_t c = n0; c < std::min(n0 + bn, n); ++c) ++cov[(size_t)r * n + c];
        }
        for(size_t i = 0; i < cov.size(); ++i)
            if(cov[i] != 1) return fail("output not covered exactly once", (long)e, (long)i);
    }
    return 0;
}

// argv[1]: random cases (default 800; the sanitizer build runs fewer)
int main(int argc, char** argv)
{
    const int iters = argc > 1 ? std::atoi(argv[1]) : 800;
    using Main     = Cfg<256, 256, 128, 2, 2, 4, 4, 16>;
    using MainWide = Cfg<128, 512, 128, 2, 1, 8, 4, 16>;
    using Silu     = Cfg<256, 256, 128, 2, 4, 2, 4, 16>;
    using SiluWide = Cfg<128, 512, 128, 2, 2, 4, 4, 16>;
    using Mid      = Cfg<128, 256, 128, 3, 2, 4, 4, 16>;
    std::mt19937   rng(20261202);
    const uint32_t special[] = {0, 1, 31, 32, 127, 128, 129, 200, 255, 256, 257, 383, 384, 385,
                                511, 512, 513, 1000, 1024, 1025, 1056, 1152, 1153};
    const uint32_t ns[]      = {256, 300, 512, 768, 1000, 1536, 2048};
    const uint32_t cuss[]    = {256, 80, 7, 2, 0};
    long           cases     = 0;
    for(int it = 0; it < iters; ++it) {
        const size_t          E = 1 + rng() % 24;
        std::vector<uint32_t> rows(E);
        for(auto& r : rows)
            r = rng() % 3 == 0 ? special[rng() % (sizeof(special) / sizeof(special[0]))]
                               : rng() % 1300;
        const uint32_t n     = ns[rng() % (sizeof(ns) / sizeof(ns[0]))];
        const uint32_t nk    = 1 + rng() % 120;
        const uint32_t cus   = cuss[rng() % (sizeof(cuss) / sizeof(cuss[0]))];
        const bool     split = rng() % 4 != 0;
        if(check<Main, MainWide>(rows, n, nk, cus, split, cases++)) return 1;
        if(check<Silu, SiluWide>(rows, n, nk, cus, split, cases++)) return 1;
        if(check<Main, Main>(rows, n, nk, cus, split, cases++)) return 1;
        if(check<Mid, Mid>(rows, n, nk, cus, split, cases++)) return 1;
    }
    // many W tiles and few C tiles: splits that cut W tiles
    for(uint32_t c = 0; c < 200; ++c) {
        std::vector<uint32_t> rows(64, 100);
        rows[0] = 256 * (1 + c % 3);
        if(check<Main, MainWide>(rows, 512 * (1 + c % 5), 64, 256, true, cases++)) return 1;
    }
    std::printf("OK %ld\n", cases);
    return 0;
}
