// Host check of the stream-K schedule arithmetic (SkPlan in
// gemm_i8_streamk_kernel.hpp), compiled and run by test_streamk_plan_cpu.py.
//
// For every (tiles, k-tiles per tile, blocks) case it walks the block ranges
// the way the kernel does and checks, by brute force:
//   * every k-tile of every tile is covered by exactly one block;
//   * pieces(t) equals the number of blocks whose range meets tile t, and
//     block_of(i) is the block whose range holds k-tile i;
//   * the slot bases (the kernel's count of cut blocks starting before the
//     tile) give each tile pieces(t) - 1 consecutive slots, disjoint from the
//     other tiles' and ending exactly at sk_slots(plan);
//   * a block meets at most two partly covered tiles;
//   * max_pieces() equals the largest pieces(t).
// Prints "OK <cases>" on success, the first failure otherwise (status 1).
#include "../optimized_rocwmma_samples_amd/csrc/gemm_i8_streamk_kernel.hpp"

#include <algorithm>
#include <cstdio>
#include <vector>

using w8a8::gemm::SkPlan;

static int fail(const SkPlan& s, const char* what, uint64_t a, uint64_t b)
{
    std::printf("FAIL tiles=%u nk=%u blocks=%u: %s (%llu, %llu)\n", s.ntiles, s.nk, s.blocks,
                what, (unsigned long long)a, (unsigned long long)b);
    return 1;
}

static int check(const SkPlan& s)
{
    const uint64_t       T = s.total();
    std::vector<int32_t> owner(T, -1);
    std::vector<std::vector<uint32_t>> touch(s.ntiles);
    for(uint32_t b = 0; b < s.blocks; ++b) {
        const uint64_t lo = s.start(b), hi = s.start(b + 1);
        if(hi <= lo) return fail(s, "empty block range", b, lo);
        uint32_t partial = 0;
        for(uint64_t it = lo; it < hi;) { // the kernel's segment walk
            const uint32_t t  = (uint32_t)(it / s.nk);
            const uint32_t k0 = (uint32_t)(it - (uint64_t)t * s.nk);
            const uint32_t k1 = (uint32_t)std::min<uint64_t>(s.nk, k0 + (hi - it));
            for(uint32_t k = k0; k < k1; ++k) {
                const uint64_t i = (uint64_t)t * s.nk + k;
                if(owner[i] != -1) return fail(s, "k-tile covered twice", i, b);
                owner[i] = (int32_t)b;
            }
            touch[t].push_back(b);
            partial += (k0 != 0 || k1 != s.nk);
            it += k1 - k0;
        }
        if(partial > 2) return fail(s, "more than two partial tiles in a block", b, partial);
    }
    for(uint64_t i = 0; i < T; ++i) {
        if(owner[i] < 0) return fail(s, "k-tile not covered", i, 0);
        if(s.block_of(i) != (uint32_t)owner[i]) return fail(s, "block_of", i, s.block_of(i));
    }
    uint32_t expect_base = 0, most = 1;
    for(uint32_t t = 0; t < s.ntiles; ++t) {
        if(s.pieces(t) != touch[t].size()) return fail(s, "pieces", t, s.pieces(t));
        most = std::max<uint32_t>(most, (uint32_t)touch[t].size());
        uint32_t base = 0; // the kernel's count: cut blocks starting before the tile
        for(uint32_t b = 1; b < s.blocks; ++b)
            base += s.cut(b) && s.start(b) < (uint64_t)t * s.nk;
        if(base != expect_base) return fail(s, "slot base", t, base);
        expect_base += s.pieces(t) - 1;
    }
    if(expect_base != w8a8::gemm::sk_slots(s)) return fail(s, "sk_slots", expect_base, 0);
    if(s.max_pieces() != most) return fail(s, "max_pieces", s.max_pieces(), most);
    return 0;
}

int main()
{
    int cases = 0;
    // the shapes the library plans: 256 CUs; cfg3's tail rounds and whole
    // problems at K = 4096 / 14336 (32 / 112 k-tiles)
    const uint32_t fixed[][3] = {{128, 32, 256}, {192, 32, 256}, {48, 32, 256}, {224, 32, 256},
                                 {32, 112, 256}, {4, 32, 128},   {16, 32, 256}, {896, 32, 256},
                                 {64, 112, 256}, {1, 1, 1},      {3, 5, 7}};
    for(const auto& f : fixed) {
        if(check(SkPlan{f[1], f[0], f[2]})) return 1;
        ++cases;
    }
    // every small combination with blocks <= tiles * nk
    for(uint32_t tiles = 1; tiles <= 40; ++tiles)
        for(uint32_t nk = 1; nk <= 24; ++nk)
            for(uint32_t blocks = 1; blocks <= 96 && blocks <= tiles * nk; ++blocks) {
                if(check(SkPlan{nk, tiles, blocks})) return 1;
                ++cases;
            }
    std::printf("OK %d\n", cases);
    return 0;
}
