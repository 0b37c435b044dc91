// w8a8_internal.hpp -- launchers shared between the kernel files and the C ABI.
// Callers (capi.cpp) have validated every argument before these run.
#pragma once

#include "../../include/w8a8.h"

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace w8a8 {

// Describes where quantizer row `i` reads from and writes to.
struct QuantRows {
    const uint16_t* x;        // fp16 source
    const float*    s;        // smooth scale (dense: [N]; moe: [experts, N])
    int8_t*         q;        // int8 destination
    float*          r;        // row scales
    uint32_t        rows;     // number of logical rows (dense: M, moe: tokens*topk)
    uint32_t        n;        // row length
    uint32_t        ldx, ldq; // strides in elements
    float           qmax;
    // MoE gather (all NULL / 0 for the dense quantizer)
    const int32_t* topk_ids;
    const int32_t* dst_row;
    uint32_t       rows_out; // destination rows (bound for dst_row entries)
    uint32_t       topk;
    uint32_t       experts;
};

hipError_t launch_smoothquant(const QuantRows& p, hipStream_t stream);

// RMSNorm (+ residual add) fused with the quantizer (rmsnorm_sq.hip).  x,
// residual and x_out share the row stride ldx; residual, x_out, y, s, q and r
// may be NULL as w8a8_add_rmsnorm_smoothquant documents.
struct NormRows {
    const uint16_t* x;
    const uint16_t* res;
    const float*    gamma;
    const float*    s;
    uint16_t*       x_out;
    uint16_t*       y;
    int8_t*         q;
    float*          r;
    uint32_t        rows, n, ldx, ldy, ldq;
    float           eps, qmax;
};
hipError_t launch_rmsnorm_sq(const NormRows& p, hipStream_t stream);

struct GemmArgs {
    uint32_t       m, n, k;
    const int8_t*  a;
    const int8_t*  b;
    void*          c;
    uint32_t       lda, ldb, ldc;
    const float*   scale_a;
    const float*   scale_b;
    float          tsa, tsb;
    int            out_type; // W8A8_OUT_*
};

// A row-major [m,k], B [n,k] K-contiguous.  Fast path requirements (checked by
// the caller through gemm_fast_path_ok): 16-byte aligned a/b, lda/ldb % 16 == 0,
// k % 16 == 0.
// Small m (decode) is routed to the decode kernel inside launch_gemm_nk.
bool       gemm_fast_path_ok(const GemmArgs& g);
// ws (optional): int32 partials of a K split, used when the launch's tiles
// fill at most half the CUs and ws_bytes >= gemm_nk_workspace_bytes(g).
hipError_t launch_gemm_nk(const GemmArgs& g, void* ws, size_t ws_bytes, hipStream_t stream);
size_t     gemm_nk_workspace_bytes(const GemmArgs& g);
// Explicit stream-K over every tile (w8a8_gemm_streamk): `blocks` blocks (0:
// one per CU, never more than the problem's k-tiles); ws: 16-byte aligned,
// streamk_workspace_bytes.  Needs gemm_fast_path_ok and A, B under 2 GiB
// (streamk_shape_ok).
bool       streamk_shape_ok(const GemmArgs& g);
size_t     streamk_workspace_bytes(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks);
uint32_t   streamk_blocks(uint32_t m, uint32_t n, uint32_t k, uint32_t blocks);
hipError_t launch_gemm_streamk(const GemmArgs& g, uint32_t blocks, void* ws, hipStream_t stream);
// The current device's stream-K status word (gemm::kSkWaitExpired bits),
// read after a device-wide synchronisation, cleared when `clear`.
hipError_t streamk_status(uint32_t* flags, bool clear);
// Test hook of the stream-K wait: polls before giving up (0: the default)
// and phantom pieces the last piece also waits for (0: none).
void       streamk_debug_wait(uint32_t spin, uint32_t phantom);
// Device address of the current GPU's W8A8_NOALLOC_SCRATCH_BYTES scratch
// array (resolved once per device; gemm_i8.hip).
hipError_t noalloc_scratch(void** ptr);

// Decode kernel (m <= kDecodeMaxM): weights streamed once, split-K across the
// waves of a block.  `packed`: g.b holds packed weights (g.ldb unused).
constexpr uint32_t kDecodeMaxM = 64;
bool       gemm_decode_ok(const GemmArgs& g);
// The decode kernel with the activation quantization folded in (packed
// weights, fp16 output, m = 1 when decode_fuse_ok): x fp16 [m, ldx] (16-byte
// aligned rows), s [k] (16-byte aligned); q [m, k] and r [m] are written as
// by the quantizer, and g.a = q, g.scale_a = r.
struct FuseArgs {
    const uint16_t* x;
    const float*    s;
    int8_t*         q;
    float*          r;
    uint32_t        ldx;
    float           qmax;
};
bool       decode_fuse_ok(uint32_t m, uint32_t k);
hipError_t launch_gemm_decode_fused(const GemmArgs& g, const FuseArgs& f, hipStream_t stream);
hipError_t launch_gemm_decode(const GemmArgs& g, bool packed, void* ws, size_t ws_bytes,
                              hipStream_t stream);

// Packed weights: [n, k] int8 rearranged into MFMA register order, 64-row
// slabs x 128-deep k-tiles of 8 KiB, zero padded (n to 64, k to 128).
size_t     packed_weight_bytes(uint32_t n, uint32_t k);
hipError_t launch_pack_weights(const int8_t* w, uint32_t n, uint32_t k, uint32_t ldw,
                               int8_t* packed, hipStream_t stream);
// Fold + per-channel quantization of fp16 weights (weights.hip); packed:
// write the packed layout (zero padding included), else row-major [n, ldq].
struct WeightQuant {
    const uint16_t* w;
    const float*    s;
    int8_t*         q;
    float*          sb;
    uint32_t        n, k, ldw, ldq;
    float           qmax;
};
hipError_t launch_quantize_weights(const WeightQuant& p, bool divide, bool packed,
                                   hipStream_t stream);

// GEMM over packed weights (g.ldb unused).  gemm_packed_ok: 16-byte aligned
// A, lda % 16 == 0, k % 16 == 0 and every A panel addressable (< 2 GiB).
bool       gemm_packed_ok(const GemmArgs& g);
hipError_t launch_gemm_packed(const GemmArgs& g, void* ws, size_t ws_bytes, hipStream_t stream);
// Split-K workspace the packed path can use for this problem (decode shapes
// 32 < m <= 64); 0 when none is used.  A smaller (or no) workspace falls back
// to the unsplit decode kernel.
size_t     packed_workspace_bytes(const GemmArgs& g);

// Generic strided GEMM (any layout/alignment): A(m,k) = a[m*sam + k*sak],
// B(n,k) = b[n*sbn + k*sbk].  Slow; used for odd shapes.
hipError_t launch_gemm_generic(const GemmArgs& g, size_t sam, size_t sak, size_t sbn,
                               size_t sbk, hipStream_t stream);

// Transposing repack: dst[r, c] = src[c*lds_src + r] for r < rows, c < cols,
// dst row-major with leading dimension ldd (zero-padded up to ldd).
hipError_t launch_transpose_i8(const int8_t* src, uint32_t lds_src, int8_t* dst, uint32_t ldd,
                               uint32_t rows, uint32_t cols, hipStream_t stream);

// ---- MoE (moe.hip) ----------------------------------------------------------
hipError_t launch_topk_softmax(const void* logits, bool f16, float* w, int32_t* ids,
                               uint32_t tokens, uint32_t experts, uint32_t topk,
                               hipStream_t stream);

size_t     moe_sort_lds_bytes(uint32_t experts);
// ws (optional, moe_sort_workspace_bytes): the multi-block sort for inputs of
// more than one block of pairs; NULL or smaller: one workgroup.
size_t     moe_sort_workspace_bytes(uint32_t tokens, uint32_t topk, uint32_t experts);
hipError_t launch_moe_sort(const int32_t* ids, uint32_t tokens, uint32_t topk, uint32_t experts,
                           uint32_t unit, int32_t* count, int32_t* start, int32_t* padded,
                           int32_t* sorted_ids, uint32_t sorted_cap, int32_t* dst_row, void* ws,
                           size_t ws_bytes, hipStream_t stream);

hipError_t launch_silu_mul_quant(const uint16_t* gu, uint32_t ld_gu, const float* s2,
                                 const int32_t* expert_start, const int32_t* expert_count,
                                 uint32_t experts, uint32_t rows, uint32_t inter, int8_t* q,
                                 uint32_t ldq, float* r, float qmax, hipStream_t stream);

hipError_t launch_moe_combine(const uint16_t* y, uint32_t ldy, uint32_t rows_y, const float* w,
                              const int32_t* dst_row, uint32_t tokens, uint32_t topk, uint32_t n,
                              uint16_t* out, uint32_t ldo, hipStream_t stream);

// Grouped GEMM over device descriptors (validated by the caller: fast-path
// alignment, every operand under 2 GiB).
// Grouped GEMM tile configurations: 0 = 256 x 256, 1 = 128 x 256, 2 = 128 x 128.
uint32_t   grouped_gemm_tiles(uint32_t m, uint32_t n, int cfg);
// The tallest configuration whose tile total is at least 3/4 of a round of
// the CUs (tiles[c] = total tiles of configuration c), else 128 x 128.
int        grouped_gemm_cfg(const uint64_t tiles[3]);
hipError_t launch_grouped_gemm(const w8a8_group_desc* groups_dev, uint32_t ngroups,
                               uint32_t total_tiles, int cfg, int out_type, int vec_ok,
                               hipStream_t stream);

struct MoeGemmArgs {
    const int8_t*  a;
    const int8_t*  w;
    void*          c;
    const float*   scale_a;
    const float*   scale_w;
    const int32_t* expert_start;
    const int32_t* expert_count;
    uint32_t       rows, experts, n, k, lda, ldw, ldc;
    uint64_t       w_stride;
    float          tsa, tsb;
    int            out_type;
    void*          ws;       // tail-split partials, or null (no split)
    size_t         ws_bytes;
};
hipError_t launch_moe_gemm(const MoeGemmArgs& a, hipStream_t stream);
// Workspace that lets launch_moe_gemm split its last partial round of tiles
// along K (one int32 tile partial per CU of the current device).
size_t moe_gemm_workspace_bytes();

// The gate_up expert GEMM with the SiLU(gate) * up epilogue, then the
// requantization of the fp16 activation (w8a8_moe_gate_up_silu).  w: the
// interleaved gate_up weights [experts, 2 * inter, k]; ws: 256-byte aligned,
// moe_gate_up_silu_workspace_bytes (activation, row maxima, split partials).
struct MoeSiluArgs {
    const int8_t*  a;
    const int8_t*  w;
    const float*   scale_a;
    const float*   scale_w; // [experts, 2 * inter], interleaved like w
    const float*   s2;      // [experts, inter] or null
    const int32_t* expert_start;
    const int32_t* expert_count;
    uint32_t       rows, experts, inter, k, lda;
    float          tsa, tsb;
    int8_t*        q;
    uint32_t       ldq;
    float*         r;
    float          qmax;
    void*          ws;
};
size_t     moe_gate_up_silu_workspace_bytes(uint32_t rows, uint32_t inter);
hipError_t launch_moe_gate_up_silu(const MoeSiluArgs& a, hipStream_t stream);
hipError_t launch_moe_interleave_gate_up(const int8_t* w, const float* sw, uint32_t experts,
                                         uint32_t inter, uint32_t k, uint32_t ldw, int8_t* wo,
                                         float* swo, hipStream_t stream);

} // namespace w8a8
