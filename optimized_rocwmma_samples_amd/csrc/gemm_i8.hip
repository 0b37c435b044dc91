// gemm_i8.hip -- launchers of the int8 GEMM: the gfx950 MFMA tile kernel
// (gemm_i8_kernel.hpp), the decode kernel for m <= 64 (gemm_i8_decode_kernel.hpp),
// the packed-weight tile kernel (gemm_i8_pb_kernel.hpp), a generic strided
// kernel for shapes the tile kernels do not take (k % 16 != 0, unaligned
// operands) and the repack used for the reference sample's A col-major /
// B [K,N] layout.
#include "gemm_i8_decode_kernel.hpp"
#include "gemm_i8_decode_wide_kernel.hpp"
#include "gemm_i8_kernel.hpp"
#include "gemm_i8_pb_kernel.hpp"
#include "gemm_i8_persist_kernel.hpp"
#include "gemm_i8_streamk_kernel.hpp"
#include "w8a8_internal.hpp"

#include <algorithm>
#include <atomic>
#include <map>
#include <mutex>
#include <tuple>

namespace w8a8 {

namespace {

using gemm::KArgs;

// Production tile configuration, and the smaller tiles of launches that
// would leave most CUs idle with it (pick_tile_cfg).  All on the
// 16 x 16 x 64 MFMA (gemm::Cfg): against the 32 x 32 x 32 form, GEMM-only,
// cold weights, cfg3 projections: M = 8192 1448 -> 1389 µs, M = 2048 411 ->
// 398 µs, M = 512 144 -> 132 µs (sum of the four).
using GemmMain  = gemm::Cfg<256, 256, 128, 2, 2, 4, 4, 16>;
// 3 LDS stages: these launches have few tiles per CU and read their panels
// from HBM, where a third k-tile in flight hides the latency (cold weights,
// M = 512: 128 x 128 o_proj 32 -> 22 µs, down 100 -> 66 µs; M = 2048,
// 128 x 256: o_proj 47 -> 40 µs, down 146 -> 116 µs).
using GemmMidM  = gemm::Cfg<128, 256, 128, 3, 2, 4, 4, 16>; // 8 waves of 64 x 64, 144 KiB LDS
using GemmSmall = gemm::Cfg<128, 128, 128, 3, 2, 4, 4, 16>; // 8 waves of 64 x 32, 96 KiB LDS
// m <= 64 over row-major weights (tiles_beat_decode): 4 waves of 64 x 32,
// 4 stages (96 KiB LDS), one tile row.
using GemmDecTile = gemm::Cfg<64, 128, 128, 4, 1, 4, 1, 16>;
// Packed-weight tile configurations (m > kDecodeMaxM): 256 x 256 blocks, and
// 128 / 64-row blocks for launches that would leave most CUs idle with them
// (pick_packed_cfg).
using GemmPacked    = gemm::PbCfg<256, 4, 2, 4>;
using GemmPacked128 = gemm::PbCfg<128, 4, 2, 4>;
using GemmPacked64  = gemm::PbCfg<64, 4, 2, 4>;
// Decode configurations: <32-row m tiles, 32-row weight tiles, waves, ring>.
using DecSmall   = gemm::DecCfg<1, 1, 4, 3>; // m <= 32, or <= 16 packed
using DecSmallW  = gemm::DecCfg<1, 2, 8, 3>; // packed, 8 <= m <= 32, many slabs
using DecMid     = gemm::DecCfg<2, 1, 8, 3>; // 32 < m <= 64
using DecMidW    = gemm::DecCfg<2, 2, 8, 2>; // packed, 32 < m <= 64, many slabs
// packed, 32 < m <= 64 with a split-K workspace: 8 half slabs per block share
// the A k-tile through LDS
using DecWide    = gemm::DecWideCfg<8, 3>;
// 4 waves of 32 weight rows: twice the blocks of DecWide, so half its K
// splits for the same fill (fewer partials; none where DecWide needs 2):
// M = 64, W [28672, 8192] 55.5 -> 49.9 us, W [8192, 28672] 59.0 -> 56.3 us.
using DecWide4   = gemm::DecWideCfg<4, 4>;
// A packed GEMM with at least this many 64-row slabs has enough blocks at
// 64 rows per block to fill the chip; fewer slabs run 32 rows per block.
constexpr uint32_t kWideSlabs = 384;

// ---------------------------------------------------------------------------
// Generic strided kernel: one thread per output, any layout / alignment.
// ---------------------------------------------------------------------------
template <int OUT>
__global__ void __launch_bounds__(256) gemm_i8_generic_kernel(KArgs p, size_t sam, size_t sak,
                                                              size_t sbn, size_t sbk)
{
    const uint32_t n = blockIdx.x * 16 + (threadIdx.x & 15);
    const uint32_t m = blockIdx.y * 16 + (threadIdx.x >> 4);
    if(m >= p.m || n >= p.n) return;
    int32_t acc = 0;
    for(uint32_t k = 0; k < p.k; ++k)
        acc += (int32_t)p.a[m * sam + k * sak] * (int32_t)p.b[n * sbn + k * sbk];
    if constexpr(OUT == W8A8_OUT_I32) {
        reinterpret_cast<int32_t*>(p.c)[(size_t)m * p.ldc + n] = acc;
    } else {
        float f = (float)acc;
        if(p.sa == nullptr && p.sb == nullptr)
            f = f * (p.tsa * p.tsb);
        else
            f = (f * (p.sa ? p.sa[m] : p.tsa)) * (p.sb ? p.sb[n] : p.tsb);
        reinterpret_cast<uint16_t*>(p.c)[(size_t)m * p.ldc + n] = float_to_half_bits_2step(f);
    }
}

__global__ void __launch_bounds__(256) transpose_i8_kernel(const int8_t* src, uint32_t lds_src,
                                                           int8_t* dst, uint32_t ldd,
                                                           uint32_t rows, uint32_t cols, int vec)
{
    // dst[r, c] = src[c * lds_src + r] (0 for c >= cols: the K padding), one
    // 64 x 64 tile per block through LDS.  Each thread moves 16 bytes each
    // way: a 16-byte run of one source row in, a 16-byte run of one
    // destination row out (vec: src and lds_src 16-byte aligned; dst and ldd
    // are, by construction).  Rows of the LDS tile are padded to 68 bytes.
    constexpr int kPitch = 68;
    __shared__ __attribute__((aligned(16))) int8_t tile[64 * kPitch];
    const uint32_t r0 = blockIdx.x * 64, c0 = blockIdx.y * 64;
    const int      t  = threadIdx.x;
    {
        const int      cl = t / 4, rc = (t % 4) * 16; // source row c0 + cl, bytes r0 + rc ..
        const uint32_t cc = c0 + cl, rr = r0 + rc;
        int4           v  = make_int4(0, 0, 0, 0);
        if(cc < cols) {
            const int8_t* p = src + (size_t)cc * lds_src + rr;
            if(vec && rr + 16 <= rows) {
                v = *reinterpret_cast<const int4*>(p);
            } else {
                int8_t b[16];
                for(int e = 0; e < 16; ++e) b[e] = rr + e < rows ? p[e] : 0;
                v = *reinterpret_cast<const int4*>(b);
            }
        }
        int* row = reinterpret_cast<int*>(tile + cl * kPitch + rc);
        row[0] = v.x;
        row[1] = v.y;
        row[2] = v.z;
        row[3] = v.w;
    }
    __syncthreads();
    const int      rl = t / 4, cc0 = (t % 4) * 16; // destination row r0 + rl, columns c0 + cc0 ..
    const uint32_t rr = r0 + rl;
    if(rr >= rows) return;
    uint32_t w[4];
#pragma unroll
    for(int q = 0; q < 4; ++q) {
        uint32_t x = 0;
#pragma unroll
        for(int e = 0; e < 4; ++e)
            x |= (uint32_t)(uint8_t)tile[(cc0 + q * 4 + e) * kPitch + rl] << (8 * e);
        w[q] = x;
    }
    const uint32_t cbase = c0 + cc0;
    int8_t*        d     = dst + (size_t)rr * ldd + cbase;
    if(cbase + 16 <= ldd) {
        *reinterpret_cast<int4*>(d) = make_int4((int)w[0], (int)w[1], (int)w[2], (int)w[3]);
    } else {
        for(int e = 0; cbase + e < ldd; ++e) d[e] = (int8_t)(w[e / 4] >> (8 * (e % 4)));
    }
}

KArgs make_kargs(const GemmArgs& g)
{
    return KArgs{g.a,   g.b,   g.c,   g.scale_a, g.scale_b, g.m,   g.n,
                 g.k,   g.lda, g.ldb, g.ldc,     g.tsa,     g.tsb};
}

int out_vec_ok(const GemmArgs& g)
{
    const size_t esz = g.out_type == W8A8_OUT_I32 ? 4 : 2;
    return (reinterpret_cast<uintptr_t>(g.c) % (4 * esz) == 0) && (g.ldc % 4 == 0)
           && (g.scale_b == nullptr || reinterpret_cast<uintptr_t>(g.scale_b) % 16 == 0);
}

// Sub-problem of rows [n0, n0 + nn) of the weights.  For packed weights n0 is
// a multiple of the 64-row slab and b points at the slab's packed block.
KArgs n_panel(const GemmArgs& g, uint32_t n0, uint32_t nn, bool packed)
{
    const size_t esz = g.out_type == W8A8_OUT_I32 ? 4 : 2;
    KArgs        p   = make_kargs(g);
    p.n              = nn;
    p.b = packed ? g.b + (size_t)(n0 / gemm::kSlab) * gemm::packed_ktiles(g.k) * gemm::kPackFrags * 1024
                 : g.b + (size_t)n0 * g.ldb;
    p.c  = static_cast<int8_t*>(g.c) + (size_t)n0 * esz;
    p.sb = g.scale_b ? g.scale_b + n0 : nullptr;
    return p;
}

// Weight rows per launch so that every buffer resource stays under 2 GiB
// (a multiple of the 64-row slab).
uint32_t weight_panel_rows(const GemmArgs& g, bool packed)
{
    constexpr size_t kLimit = 0x7FFFFFFFull;
    size_t           rows;
    if(packed)
        rows = kLimit / ((size_t)gemm::packed_ktiles(g.k) * gemm::kPackFrags * 1024) * gemm::kSlab;
    else
        rows = (kLimit - g.k) / g.ldb + 1;
    rows = std::max<size_t>(gemm::kSlab, rows / gemm::kSlab * gemm::kSlab);
    return (uint32_t)std::min<size_t>(g.n, rows);
}

uint32_t device_cus()
{
    static const uint32_t cus = [] {
        int dev = 0, c = 256;
        if(hipGetDevice(&dev) == hipSuccess)
            (void)hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev);
        return (uint32_t)c;
    }();
    return cus;
}

// Tile configuration of one launch.  256 x 256 tiles have the best per-op
// rate once they fill the chip; a launch with fewer than 3/4 of a round of
// them leaves most CUs idle, and smaller tiles finish it sooner (measured
// on MI355X, cfg3 shapes: M = 512 qkv 46 -> 25 µs, o_proj 45 -> 22 µs,
// down 140 -> 71 µs with 128 x 128; M = 2048 o_proj 59 -> 42 µs, down
// 164 -> 119 µs with 128 x 256; the shapes with enough 256 x 256 tiles, e.g.
// M = 2048 qkv or gate_up, are slower with smaller ones).
enum class TileCfg { kMain, kMidM, kSmall, kDecode };

TileCfg pick_tile_cfg(uint32_t m, uint32_t n)
{
    if(m <= kDecodeMaxM) return TileCfg::kDecode;
    auto tiles = [&](uint32_t bm, uint32_t bn) {
        return (uint64_t)((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    };
    const uint64_t enough = (uint64_t)device_cus() * 3 / 4;
    if(tiles(GemmMain::kBM, GemmMain::kBN) >= enough) return TileCfg::kMain;
    if(tiles(GemmMidM::kBM, GemmMidM::kBN) >= enough) return TileCfg::kMidM;
    return TileCfg::kSmall;
}

// Block height of a packed-weight launch (blocks are always 256 weight
// columns): the tallest of 256 / 128 / 64 rows that gives at least 3/4 of a
// round of blocks, else 64.
int pick_packed_cfg(uint32_t m, uint32_t n)
{
    const uint64_t cols   = (n + GemmPacked::kBN - 1) / GemmPacked::kBN;
    const uint64_t enough = (uint64_t)device_cus() * 3 / 4;
    if((m + 255) / 256 * cols >= enough) return 256;
    if((m + 127) / 128 * cols >= enough) return 128;
    return 64;
}

// K split of a dense launch (one panel): when the chosen tiles fill at most
// half of the CUs, each tile runs as `parts` K pieces on otherwise idle CUs
// (gemm_i8_split_kernel + fixup).  parts = 1: no split.
struct DenseSplit {
    TileCfg  cfg;
    uint32_t tiles, parts;
    size_t   bytes; // workspace the split needs
};

DenseSplit dense_split(uint32_t m, uint32_t n, uint32_t k)
{
    DenseSplit d{pick_tile_cfg(m, n), 0, 1, 0};
    uint32_t   bm = GemmMain::kBM, bn = GemmMain::kBN;
    size_t     part_bytes = gemm::Partial<GemmMain>::kBytes;
    if(d.cfg == TileCfg::kMidM) {
        bm = GemmMidM::kBM, bn = GemmMidM::kBN, part_bytes = gemm::Partial<GemmMidM>::kBytes;
    } else if(d.cfg == TileCfg::kSmall) {
        bm = GemmSmall::kBM, bn = GemmSmall::kBN, part_bytes = gemm::Partial<GemmSmall>::kBytes;
    } else if(d.cfg == TileCfg::kDecode) {
        bm = GemmDecTile::kBM, bn = GemmDecTile::kBN,
        part_bytes = gemm::Partial<GemmDecTile>::kBytes;
    }
    d.tiles             = ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    const uint32_t cus  = device_cus();
    const uint32_t nk   = (k + 127) / 128;
    if((uint64_t)d.tiles * 2 > cus) return d;
    const uint32_t parts = std::min({cus / d.tiles, nk / gemm::kMinKtPerPart, gemm::kMaxParts});
    if(parts < 2) return d;
    d.parts = parts;
    d.bytes = (size_t)d.tiles * parts * part_bytes;
    return d;
}

// K splits of the wide decode kernel for one weight panel: the count that
// minimises the weight bytes of the busiest CU, ceil(blocks / CUs) / splits
// (the fewest splits among equals), at least 8 k-tiles per split; 1 = no
// split.  E.g. 112 panels of W1 on 256 CUs: 2 splits (224 blocks, one per
// CU) rather than 3 (336 blocks: 80 CUs would stream two).
uint32_t decode_wide_splits(const GemmArgs& g, uint32_t n)
{
    const uint32_t cus  = device_cus();
    const uint32_t nblk = (n + DecWide::kRows - 1) / DecWide::kRows;
    const uint32_t nkt  = gemm::packed_ktiles(g.k);
    const uint32_t most = std::max<uint32_t>(1, std::min<uint32_t>(nkt / 8, 8));
    uint32_t       best = 1;
    double         cost = 1e30;
    for(uint32_t s = 1; s <= most; ++s) {
        const double c = (double)((nblk * s + cus - 1) / cus) / s;
        if(c < cost * (1 - 1e-9)) {
            cost = c;
            best = s;
        }
    }
    return best;
}

bool decode_wide_shape(const GemmArgs& g) { return g.m > 32 && g.m <= kDecodeMaxM; }

} // namespace

size_t packed_workspace_bytes(const GemmArgs& g)
{
    if(!decode_wide_shape(g) || !gemm_decode_ok(g)) return 0;
    const uint32_t step = weight_panel_rows(g, true);
    size_t         most = 0;
    for(uint32_t n0 = 0; n0 < g.n; n0 += step) {
        const uint32_t nn = std::min(step, g.n - n0);
        most = std::max(most, gemm::decode_ws_bytes(g.m, nn, decode_wide_splits(g, nn)));
    }
    return most;
}

bool gemm_decode_ok(const GemmArgs& g)
{
    return g.m <= kDecodeMaxM && (uint64_t)(g.m - 1) * g.lda + g.k < 0x7FFFFFFFull;
}

// The row quantized inside the decode kernel (w8a8_fused_sq_gemm_packed at
// m <= kFuseRows = 1 and k <= kFuseMaxK): every block quantizes the row
// before its A-dependent MFMAs, a prologue that grows with K.  It pays where
// it is short and saves the quantizer launch: M = 1, N = K = 4096 8.9 ->
// 7.2 us, N = K = 1024 5.7 -> 4.1 us, [14336, 4096] 13.8 -> 12.0 us, W1
// [28672, 8192] level (41.8 / 41.7 us); at W2 [8192, 28672] (one block per
// CU, 28672-element rows) it cost 48.9 -> 54.5 us, so longer rows keep the
// separate quantizer.
constexpr uint32_t kFuseMaxK = 8192;
bool decode_fuse_ok(uint32_t m, uint32_t k)
{
    const uint64_t pitch = (uint64_t)gemm::packed_ktiles(k) * gemm::kPackK + gemm::kFusePad;
    return m >= 1 && m <= gemm::kFuseRows && k <= kFuseMaxK
           && DecSmall::kLdsBytes + m * pitch <= 160 * 1024;
}

hipError_t launch_gemm_decode_fused(const GemmArgs& g, const FuseArgs& f, hipStream_t stream)
{
    const uint32_t    ka = gemm::packed_ktiles(g.k) * gemm::kPackK;
    const gemm::FuseQ fq{f.x, f.s, f.q, f.r, f.ldx, ka, ka + gemm::kFusePad, f.qmax};
    const int      vec_ok = out_vec_ok(g);
    const uint32_t step   = weight_panel_rows(g, true);
    for(uint32_t n0 = 0; n0 < g.n; n0 += step) {
        const KArgs      p = n_panel(g, n0, std::min(step, g.n - n0), true);
        const hipError_t e = gemm::launch_decode_fused<DecSmall>(p, fq, vec_ok, stream);
        if(e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_gemm_decode(const GemmArgs& g, bool packed, void* ws, size_t ws_bytes,
                              hipStream_t stream)
{
    if(g.m == 0 || g.n == 0) return hipSuccess;
    const int      vec_ok = out_vec_ok(g);
    const uint32_t step   = weight_panel_rows(g, packed);
    const bool     wide   = packed && gemm::packed_slabs(g.n) >= kWideSlabs;
    for(uint32_t n0 = 0; n0 < g.n; n0 += step) {
        const KArgs p = n_panel(g, n0, std::min(step, g.n - n0), packed);
        hipError_t  e;
        if(packed && decode_wide_shape(g) && ws != nullptr) {
            // the workspace holds every panel's partials (panels run in stream order)
            const uint32_t splits = decode_wide_splits(g, p.n);
            // the 4-wave form: twice the blocks, so half the splits for the
            // same fill (1 = unsplit, no reduce launch)
            const uint64_t b4 = (uint64_t)(p.n + DecWide4::kRows - 1) / DecWide4::kRows * (splits / 2);
            if(splits % 2 == 0 && b4 * 4 >= (uint64_t)device_cus() * 3 && b4 <= device_cus()
               && gemm::decode_ws_bytes(g.m, p.n, splits / 2) <= ws_bytes) {
                e = gemm::launch_decode_wide<DecWide4>(p, g.out_type, vec_ok,
                                                       static_cast<int32_t*>(ws), splits / 2,
                                                       stream);
                if(e != hipSuccess) return e;
                continue;
            }
            if(gemm::decode_ws_bytes(g.m, p.n, splits) <= ws_bytes) {
                e = gemm::launch_decode_wide<DecWide>(p, g.out_type, vec_ok,
                                                      static_cast<int32_t*>(ws), splits, stream);
                if(e != hipSuccess) return e;
                continue;
            }
        }
        if(packed) {
            // 8 <= m <= 16 on many slabs: 64 weight rows per block halve the
            // re-reads of the activation rows (M=16 N=28672: 54 -> 52 us)
            if((g.m <= 16 && (!wide || g.m < 8)) || (g.m <= 32 && !wide))
                e = gemm::launch_decode<DecSmall, true>(p, g.out_type, vec_ok, stream);
            else if(g.m <= 32)
                e = gemm::launch_decode<DecSmallW, true>(p, g.out_type, vec_ok, stream);
            else if(!wide)
                e = gemm::launch_decode<DecMid, true>(p, g.out_type, vec_ok, stream);
            else
                e = gemm::launch_decode<DecMidW, true>(p, g.out_type, vec_ok, stream);
        } else {
            if(g.m <= 32)
                e = gemm::launch_decode<DecSmall, false>(p, g.out_type, vec_ok, stream);
            else
                e = gemm::launch_decode<DecMid, false>(p, g.out_type, vec_ok, stream);
        }
        if(e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_gemm_packed(const GemmArgs& g, void* ws, size_t ws_bytes, hipStream_t stream)
{
    if(g.m == 0 || g.n == 0) return hipSuccess;
    if(gemm_decode_ok(g)) return launch_gemm_decode(g, true, ws, ws_bytes, stream);
    const size_t   esz    = g.out_type == W8A8_OUT_I32 ? 4 : 2;
    const int      vec_ok = out_vec_ok(g);
    constexpr size_t kLimit = 0x7FFFFFFFull;
    const uint32_t mstep  = (uint32_t)std::min<size_t>(
        g.m, std::max<size_t>(GemmPacked::kBM, kLimit / g.lda / GemmPacked::kBM * GemmPacked::kBM));
    // the packed tile kernel's blocks cover 256 weight rows: keep panels aligned to that
    const uint32_t nstep = std::max<uint32_t>(
        GemmPacked::kBN, weight_panel_rows(g, true) / GemmPacked::kBN * GemmPacked::kBN);
    for(uint32_t m0 = 0; m0 < g.m; m0 += mstep) {
        for(uint32_t n0 = 0; n0 < g.n; n0 += nstep) {
            KArgs p = n_panel(g, n0, std::min(nstep, g.n - n0), true);
            p.m     = std::min(mstep, g.m - m0);
            p.a     = g.a + (size_t)m0 * g.lda;
            p.c     = static_cast<int8_t*>(p.c) + (size_t)m0 * g.ldc * esz;
            p.sa    = g.scale_a ? g.scale_a + m0 : nullptr;
            hipError_t e;
            switch(pick_packed_cfg(p.m, p.n)) {
            case 256: e = gemm::launch_pb<GemmPacked>(p, g.out_type, vec_ok, stream); break;
            case 128: e = gemm::launch_pb<GemmPacked128>(p, g.out_type, vec_ok, stream); break;
            default: e = gemm::launch_pb<GemmPacked64>(p, g.out_type, vec_ok, stream); break;
            }
            if(e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

size_t packed_weight_bytes(uint32_t n, uint32_t k) { return gemm::packed_bytes(n, k); }

hipError_t launch_pack_weights(const int8_t* w, uint32_t n, uint32_t k, uint32_t ldw,
                               int8_t* packed, hipStream_t stream)
{
    return gemm::launch_pack_weights(w, n, k, ldw, packed, stream);
}

bool gemm_fast_path_ok(const GemmArgs& g)
{
    // every launch addresses A and B panels of at least one tile of rows
    // through buffer resources: a tile's rows must fit in 2 GiB
    constexpr uint64_t kLimit = 0x7FFFFFFFull;
    return (reinterpret_cast<uintptr_t>(g.a) % 16 == 0)
           && (reinterpret_cast<uintptr_t>(g.b) % 16 == 0) && (g.lda % 16 == 0)
           && (g.ldb % 16 == 0) && (g.k % 16 == 0)
           && (uint64_t)g.lda * GemmMain::kBM <= kLimit && (uint64_t)g.ldb * GemmMain::kBN <= kLimit;
}

bool gemm_packed_ok(const GemmArgs& g)
{
    constexpr uint64_t kLimit = 0x7FFFFFFFull;
    if(reinterpret_cast<uintptr_t>(g.a) % 16 != 0 || g.lda % 16 != 0 || g.k % 16 != 0) return false;
    // one packed k-row of a 64-row slab must fit in 2 GiB
    if((uint64_t)gemm::packed_ktiles(g.k) * gemm::kPackFrags * 1024 > kLimit) return false;
    return g.m <= kDecodeMaxM ? gemm_decode_ok(g) : (uint64_t)g.lda * GemmPacked::kBM <= kLimit;
}

// Row-major weights at m <= 64: the decode kernel streams 32-row weight
// panels with 32-byte pieces per lane and re-reads all of A for every panel
// (at m = 64 twice the weight bytes from L2); 64 x 128 tiles load each
// weight tile once as whole 128-byte rows.  They take over when they fill
// the chip by themselves, or with a K split when the caller gave the
// workspace.  Cold weights, W [28672, 8192]: m = 1 61 -> 51 µs, m = 16
// 72 -> 54 µs, m = 32 83 -> 54 µs, m = 64 96 -> 53 µs; W [8192, 28672]
// has 64 tiles and needs the split.
bool tiles_beat_decode(const GemmArgs& g, void* ws, size_t ws_bytes)
{
    const DenseSplit d = dense_split(g.m, g.n, g.k);
    if(d.parts == 1) return d.tiles >= (uint64_t)device_cus() * 3 / 4;
    return ws != nullptr && ws_bytes >= d.bytes;
}

// The persistent tile kernel for a 256 x 256 launch: fp16 output, at least
// two tiles per CU and at most 32 k-tiles per tile.  It saves a fixed cost
// per tile (workgroup launch, cold prologue, store burst), which pays where
// tiles are short: 2-4% at M=8192 K=4096 N=28672, 10-20% at K <= 1024,
// nothing measurable at K=14336 with two tiles per CU.
bool persist_pays(const KArgs& p, int out_type, int vec_ok)
{
    return out_type == W8A8_OUT_F16 && (p.k + GemmMain::kBK - 1) / GemmMain::kBK <= 32
           && gemm::persist_ok<GemmMain>(p, vec_ok, device_cus());
}

size_t gemm_nk_workspace_bytes(const GemmArgs& g)
{
    if(g.m == 0 || g.n == 0 || g.k == 0) return 0;
    return dense_split(g.m, g.n, g.k).bytes;
}

// One 256 x 256 launch (a panel).  When its tiles make whole rounds over the
// CUs plus a last round at most half full, and the whole rounds are whole
// columns of tiles, the columns of the last round run as 128 x 256 tiles in
// a launch of their own: twice the tiles, each half the work, so that round
// keeps every CU busy for about half as long (cfg3 gate_up at M = 2048:
// 8 x 112 tiles = 3 rounds + 128 tiles; the last 16 columns become one
// round of 256 tiles of 128 x 256).  The same k-order per output, so the
// result is bit-identical to the single launch.
hipError_t launch_main(const KArgs& p, int out_type, int vec_ok, hipStream_t stream)
{
    const uint32_t cus   = device_cus();
    const uint32_t tm    = (p.m + GemmMain::kBM - 1) / GemmMain::kBM;
    const uint32_t tiles = tm * ((p.n + GemmMain::kBN - 1) / GemmMain::kBN);
    const uint32_t full = tiles / cus, rest = tiles % cus;
    const uint32_t mid_rows = (p.m + GemmMidM::kBM - 1) / GemmMidM::kBM;
    if(full >= 1 && rest > 0 && rest * 2 <= cus && (full * cus) % tm == 0) {
        const uint32_t n1   = full * cus / tm * GemmMain::kBN; // < p.n: rest > 0
        const uint32_t n2   = p.n - n1;
        const size_t   esz  = out_type == W8A8_OUT_I32 ? 4 : 2;
        if((uint64_t)mid_rows * ((n2 + GemmMidM::kBN - 1) / GemmMidM::kBN) <= cus) {
            KArgs head = p, tail = p;
            head.n     = n1;
            tail.n     = n2;
            tail.b     = p.b + (size_t)n1 * p.ldb;
            tail.c     = static_cast<int8_t*>(p.c) + (size_t)n1 * esz;
            tail.sb    = p.sb ? p.sb + n1 : nullptr;
            hipError_t e = persist_pays(head, out_type, vec_ok)
                               ? gemm::launch_cfg_persist<GemmMain>(head, vec_ok, cus, stream)
                               : gemm::launch_cfg<GemmMain>(head, out_type, vec_ok, stream);
            if(e != hipSuccess) return e;
            return gemm::launch_cfg<GemmMidM>(tail, out_type, vec_ok, stream);
        }
    }
    return persist_pays(p, out_type, vec_ok)
               ? gemm::launch_cfg_persist<GemmMain>(p, vec_ok, cus, stream)
               : gemm::launch_cfg<GemmMain>(p, out_type, vec_ok, stream);
}

hipError_t launch_gemm_nk(const GemmArgs& g, void* ws, size_t ws_bytes, hipStream_t stream)
{
    if(g.m == 0 || g.n == 0) return hipSuccess;
    if(gemm_decode_ok(g) && !tiles_beat_decode(g, ws, ws_bytes))
        return launch_gemm_decode(g, false, nullptr, 0, stream);
    const size_t esz    = g.out_type == W8A8_OUT_I32 ? 4 : 2;
    const int    vec_ok = out_vec_ok(g);
    // The tile kernel addresses each operand through a buffer resource whose
    // out-of-range offsets read as zero; keep every launch's A and B under
    // 2 GiB by splitting M and N into row panels (multiples of the tile).
    constexpr size_t kLimit = 0x7FFFFFFFull;
    const uint32_t   mstep  = (uint32_t)std::min<size_t>(
        g.m, std::max<size_t>(GemmMain::kBM, kLimit / g.lda / GemmMain::kBM * GemmMain::kBM));
    const uint32_t nstep = (uint32_t)std::min<size_t>(
        g.n, std::max<size_t>(GemmMain::kBN, kLimit / g.ldb / GemmMain::kBN * GemmMain::kBN));
    if(ws != nullptr && mstep == g.m && nstep == g.n) {
        const DenseSplit d = dense_split(g.m, g.n, g.k);
        if(d.parts > 1 && ws_bytes >= d.bytes) {
            const KArgs p  = make_kargs(g);
            int32_t*    pw = static_cast<int32_t*>(ws);
            switch(d.cfg) {
            case TileCfg::kMain:
                return gemm::launch_cfg_split<GemmMain>(p, g.out_type, vec_ok, pw, d.parts, stream);
            case TileCfg::kMidM:
                return gemm::launch_cfg_split<GemmMidM>(p, g.out_type, vec_ok, pw, d.parts, stream);
            case TileCfg::kSmall:
                return gemm::launch_cfg_split<GemmSmall>(p, g.out_type, vec_ok, pw, d.parts, stream);
            default:
                return gemm::launch_cfg_split<GemmDecTile>(p, g.out_type, vec_ok, pw, d.parts,
                                                           stream);
            }
        }
    }
    for(uint32_t m0 = 0; m0 < g.m; m0 += mstep) {
        for(uint32_t n0 = 0; n0 < g.n; n0 += nstep) {
            KArgs p = make_kargs(g);
            p.m     = std::min(mstep, g.m - m0);
            p.n     = std::min(nstep, g.n - n0);
            p.a     = g.a + (size_t)m0 * g.lda;
            p.b     = g.b + (size_t)n0 * g.ldb;
            p.c     = static_cast<int8_t*>(g.c) + ((size_t)m0 * g.ldc + n0) * esz;
            p.sa    = g.scale_a ? g.scale_a + m0 : nullptr;
            p.sb    = g.scale_b ? g.scale_b + n0 : nullptr;
            hipError_t e;
            switch(pick_tile_cfg(p.m, p.n)) {
            case TileCfg::kMain: e = launch_main(p, g.out_type, vec_ok, stream); break;
            case TileCfg::kMidM: e = gemm::launch_cfg<GemmMidM>(p, g.out_type, vec_ok, stream); break;
            case TileCfg::kSmall: e = gemm::launch_cfg<GemmSmall>(p, g.out_type, vec_ok, stream); break;
            default: e = gemm::launch_cfg<GemmDecTile>(p, g.out_type, vec_ok, stream); break;
            }
            if(e != hipSuccess) return e;
        }
    }
    return hipSuccess;
}

namespace {

// Explicit stream-K (w8a8_gemm_streamk): every tile of the problem in the
// stream-K schedule over `blocks` blocks (0: one per CU), the reference
// sample's decomposition (rocwmma_streamk_gemm.cpp:223-226).  The tile is
// the largest of 256 x 256, 128 x 256 and 128 x 128 that leaves each block
// at least 8 k-tiles (else 128 x 128); never more blocks than k-tiles.
struct ExplicitSk {
    TileCfg      cfg;
    gemm::SkPlan plan;
    size_t       bytes;
};

// Estimated critical path of a stream-K plan on tile configuration C: the
// longest block's k-tiles at C's rate per CU (`tops`, whole chip, measured on
// the dense kernels: the smaller tiles sustain less), plus the partials the
// last piece of the most-split tile reads back at `xbw` bytes/s (device-scope
// loads; fitted to the square and cfg3 CLI shapes, lower for the larger
// tiles, whose kernels spill around the exchange).  Splitting a tile over P
// blocks costs its last block P - 1 partials, so fewer, larger tiles win
// only where their pieces stay few: 2048^3 ran 75 µs on 256 x 256 tiles (4
// pieces each) against 26 µs on 128 x 128 tiles (one block per tile).
template <class C>
double sk_cost(const gemm::SkPlan& s, double tops, double xbw)
{
    const uint64_t u    = (s.total() + s.blocks - 1) / s.blocks;
    const uint32_t pmax = s.max_pieces();
    const double unit_s = 2.0 * C::kBM * C::kBN * C::kBK / (tops / device_cus());
    return (double)u * unit_s + (pmax - 1) * (double)gemm::Partial<C>::kBytes / xbw;
}

// blocks = 0: the block count is chosen too, among one per CU and 1/2, 1/4,
// 1/8 of that: a few tiles cut into many pieces cost their last blocks more
// partials than the extra blocks save (512^3: 16 pieces per tile on 256
// blocks, 4 on 64).
ExplicitSk plan_streamk(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks)
{
    const uint32_t nk = (k + 127) / 128;
    ExplicitSk     e{TileCfg::kMain, {}, 0};
    double         best = 1e300;
    for(uint32_t div = 1; div <= (blocks ? 1u : 8u); div *= 2) {
        const uint32_t G = blocks ? blocks : std::max(1u, device_cus() / div);
        auto plan = [&](uint32_t bm, uint32_t bn) {
            const uint32_t tiles = ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
            return gemm::SkPlan{nk, tiles, (uint32_t)std::min<uint64_t>(G, (uint64_t)tiles * nk)};
        };
        const ExplicitSk cand[3] = {
            {TileCfg::kMain, plan(GemmMain::kBM, GemmMain::kBN), 0},
            {TileCfg::kMidM, plan(GemmMidM::kBM, GemmMidM::kBN), 0},
            {TileCfg::kSmall, plan(GemmSmall::kBM, GemmSmall::kBN), 0}};
        const double cost[3] = {sk_cost<GemmMain>(cand[0].plan, 2.5e15, 13e9),
                                sk_cost<GemmMidM>(cand[1].plan, 2.1e15, 15e9),
                                sk_cost<GemmSmall>(cand[2].plan, 1.7e15, 35e9)};
        for(int c = 0; c < 3; ++c)
            if(cost[c] < best * (1 - 1e-9)) {
                best = cost[c];
                e    = cand[c];
            }
    }
    e.bytes = e.cfg == TileCfg::kMain   ? gemm::sk_workspace_bytes<GemmMain>(e.plan)
              : e.cfg == TileCfg::kMidM ? gemm::sk_workspace_bytes<GemmMidM>(e.plan)
                                        : gemm::sk_workspace_bytes<GemmSmall>(e.plan);
    return e;
}

// plan_streamk memoized per (m, n, k, blocks): every w8a8_gemm_streamk call
// needs the plan twice (the workspace check, then the launch) and a caller
// sizing its workspace a third time; the plan depends on nothing else (the CU
// count is the process's first device's).  The table is bounded: a caller
// cycling through more shapes than kMaxPlans starts it over.
ExplicitSk explicit_streamk(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks)
{
    constexpr size_t kMaxPlans = 1024;
    struct Key {
        uint32_t m, n, k, blocks;
        bool     operator<(const Key& o) const
        {
            return std::tie(m, n, k, blocks) < std::tie(o.m, o.n, o.k, o.blocks);
        }
    };
    static std::mutex               mu;
    static std::map<Key, ExplicitSk> plans;
    const Key                        key{m, n, k, blocks};
    {
        std::lock_guard<std::mutex> lock(mu);
        const auto                  it = plans.find(key);
        if(it != plans.end()) return it->second;
    }
    const ExplicitSk e = plan_streamk(m, n, k, blocks);
    std::lock_guard<std::mutex> lock(mu);
    if(plans.size() >= kMaxPlans) plans.clear();
    plans.emplace(key, e);
    return e;
}

} // namespace

bool streamk_shape_ok(const GemmArgs& g)
{
    constexpr uint64_t kLimit = 0x7FFFFFFFull;
    return gemm_fast_path_ok(g) && (uint64_t)g.m * g.lda <= kLimit
           && (uint64_t)g.n * g.ldb <= kLimit;
}

size_t streamk_workspace_bytes(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks)
{
    if(m == 0 || n == 0 || k == 0) return 0;
    return explicit_streamk(m, n, k, blocks).bytes;
}

uint32_t streamk_blocks(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks)
{
    if(m == 0 || n == 0 || k == 0) return 0;
    return explicit_streamk(m, n, k, blocks).plan.blocks;
}

// ---------------------------------------------------------------------------
// The stream-K wait's status word (gemm::SkWatch): one per GPU, a file-scope
// device array like the no-allocation scratch below, reached from the host
// only through the address hipGetSymbolAddress returns for the current
// device.  Zero-initialised when the code object loads; a kernel only ORs
// bits into it; streamk_status reads (and optionally clears) it.
// ---------------------------------------------------------------------------
static __device__ __align__(256) uint32_t sk_status[64];

namespace {

hipError_t sk_status_ptr(uint32_t** ptr)
{
    constexpr int     kMaxDevices = 64;
    static std::mutex mu;
    static void*      addr[kMaxDevices] = {};
    int               dev               = 0;
    hipError_t        e                 = hipGetDevice(&dev);
    if(e != hipSuccess) return e;
    if(dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if(addr[dev] == nullptr) {
        void* p = nullptr;
        e       = hipGetSymbolAddress(&p, HIP_SYMBOL(sk_status));
        if(e != hipSuccess) return e;
        addr[dev] = p;
    }
    *ptr = static_cast<uint32_t*>(addr[dev]);
    return hipSuccess;
}

// the wait's poll limit and phantom piece count (test hook only)
std::atomic<uint32_t> g_sk_spin{gemm::kSkSpinLimit};
std::atomic<uint32_t> g_sk_phantom{0};

} // namespace

void streamk_debug_wait(uint32_t spin, uint32_t phantom)
{
    g_sk_spin.store(spin ? spin : gemm::kSkSpinLimit);
    g_sk_phantom.store(phantom);
}

hipError_t streamk_status(uint32_t* flags, bool clear)
{
    uint32_t*  ptr = nullptr;
    hipError_t e   = sk_status_ptr(&ptr);
    if(e != hipSuccess) return e;
    // every launch that may set the word has finished, on any stream
    if((e = hipDeviceSynchronize()) != hipSuccess) return e;
    if((e = hipMemcpy(flags, ptr, sizeof(uint32_t), hipMemcpyDeviceToHost)) != hipSuccess) return e;
    if(clear && *flags) {
        const uint32_t zero = 0;
        e = hipMemcpy(ptr, &zero, sizeof(uint32_t), hipMemcpyHostToDevice);
    }
    return e;
}

hipError_t launch_gemm_streamk(const GemmArgs& g, uint32_t blocks, void* ws, hipStream_t stream)
{
    if(g.m == 0 || g.n == 0) return hipSuccess;
    gemm::SkWatch watch{nullptr, g_sk_spin.load(), g_sk_phantom.load()};
    const hipError_t err = sk_status_ptr(&watch.status);
    if(err != hipSuccess) return err;
    const ExplicitSk e      = explicit_streamk(g.m, g.n, g.k, blocks);
    const KArgs      p      = make_kargs(g);
    const int        vec_ok = out_vec_ok(g);
    if(e.plan.blocks == e.plan.ntiles) {
        // one whole tile per block, no pieces: the schedule is the tile
        // kernel's one-block-per-tile grid (the same logical block -> tile
        // order), which runs it without the counters' clear launch and with
        // the epilogue's scales loaded under the last k-tile
        switch(e.cfg) {
        case TileCfg::kMain: return gemm::launch_cfg<GemmMain>(p, g.out_type, vec_ok, stream);
        case TileCfg::kMidM: return gemm::launch_cfg<GemmMidM>(p, g.out_type, vec_ok, stream);
        default: return gemm::launch_cfg<GemmSmall>(p, g.out_type, vec_ok, stream);
        }
    }
    switch(e.cfg) {
    case TileCfg::kMain:
        return gemm::launch_cfg_streamk<GemmMain>(p, g.out_type, vec_ok, 0, e.plan, ws, watch,
                                                  stream);
    case TileCfg::kMidM:
        return gemm::launch_cfg_streamk<GemmMidM>(p, g.out_type, vec_ok, 0, e.plan, ws, watch,
                                                  stream);
    default:
        return gemm::launch_cfg_streamk<GemmSmall>(p, g.out_type, vec_ok, 0, e.plan, ws, watch,
                                                   stream);
    }
}

hipError_t launch_gemm_generic(const GemmArgs& g, size_t sam, size_t sak, size_t sbn, size_t sbk,
                               hipStream_t stream)
{
    if(g.m == 0 || g.n == 0) return hipSuccess;
    const KArgs p = make_kargs(g);
    dim3        grid((g.n + 15) / 16, (g.m + 15) / 16);
    if(g.out_type == W8A8_OUT_I32)
        hipLaunchKernelGGL(gemm_i8_generic_kernel<W8A8_OUT_I32>, grid, dim3(256), 0, stream, p,
                           sam, sak, sbn, sbk);
    else
        hipLaunchKernelGGL(gemm_i8_generic_kernel<W8A8_OUT_F16>, grid, dim3(256), 0, stream, p,
                           sam, sak, sbn, sbk);
    return hipGetLastError();
}

hipError_t launch_transpose_i8(const int8_t* src, uint32_t lds_src, int8_t* dst, uint32_t ldd,
                               uint32_t rows, uint32_t cols, hipStream_t stream)
{
    dim3      grid((rows + 63) / 64, (ldd + 63) / 64);
    const int vec = reinterpret_cast<uintptr_t>(src) % 16 == 0 && lds_src % 16 == 0;
    hipLaunchKernelGGL(transpose_i8_kernel, grid, dim3(256), 0, stream, src, lds_src, dst, ldd,
                       rows, cols, vec);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Scratch of w8a8_gemm_noalloc: a file-scope device array.  Every GPU that
// loads this code object holds its own copy until the process ends; host code
// uses it only through the device address hipGetSymbolAddress returns, looked
// up once per device with that device current (the array's name is a host
// stand-in, not a device address).  The K-split partials that live in it are
// written in full before they are read, so nothing is cleared between calls;
// calls that overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------
static __device__ __align__(256) int8_t scratch[W8A8_NOALLOC_SCRATCH_BYTES];

hipError_t noalloc_scratch(void** ptr)
{
    constexpr int      kMaxDevices = 64;
    static std::mutex  mu;
    static void*       addr[kMaxDevices] = {};
    int                dev               = 0;
    hipError_t         e                 = hipGetDevice(&dev);
    if(e != hipSuccess) return e;
    if(dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if(addr[dev] == nullptr) {
        void* p = nullptr;
        e       = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if(e != hipSuccess) return e;
        addr[dev] = p;
    }
    *ptr = addr[dev];
    return hipSuccess;
}

} // namespace w8a8
