"""MI355X-native W8A8 SmoothQuant path (gfx950 HIP kernels behind a C ABI).

Python layer over libw8a8.so.  Device tensors come from PyTorch (memory and
streams only); every computation runs in the hand-written HIP kernels of
libw8a8.so, enqueued on torch's current stream.  Nothing here falls back to
CPU or PyTorch math: a missing library raises.

The functions mirror the reference kernels this path replaces:
  smoothquant      <- kernel_smoothquant      (rocwmma_smoothquant.cpp:58-122)
  moe_smoothquant  <- kernel_moe_smoothquant  (rocwmma_moe_smoothquant.cpp:69-131)
  gemm             <- gemm_quant_tensor_scale (rocwmma_gemm_quantized.cpp:127-195), Mode 2
  fused_sq_gemm    <- smoothquant feeding gemm, one call
"""
from __future__ import annotations

from . import _lib
from ._lib import (  # noqa: F401
    ERROR_INVALID_VALUE,
    ERROR_NOT_SUPPORTED,
    LAYOUT_A_COL_B_KN,
    LAYOUT_A_ROW_B_NK,
    OUT_F16,
    OUT_I32,
    W8A8Error,
)

__all__ = [
    "library", "version", "smoothquant", "moe_smoothquant", "gemm", "gemm_workspace_size",
    "fused_sq_gemm", "W8A8Error",
]


def library():
    """The loaded ctypes library (raises if libw8a8.so was not built)."""
    return _lib.load()


def version() -> str:
    return library().w8a8_version().decode()


def _torch():
    import torch
    return torch


def _stream(device=None) -> int:
    torch = _torch()
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _require_cuda(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("W8A8 kernels take device tensors (got a CPU tensor)")


def smoothquant(x, smooth_scale, quant_max: float = 127.0, out=None, row_scale=None):
    """Row-wise smooth-scale + absmax int8 quantization of fp16 x [M, N].

    Returns (q int8 [M, N], row_scale fp32 [M]).  x may be row-strided
    (x.stride(1) == 1); q is written row-major (or into `out`, any row stride).
    """
    torch = _torch()
    _require_cuda(x, smooth_scale)
    if x.dim() != 2 or x.dtype != torch.float16 or x.stride(1) != 1:
        raise ValueError("x must be a 2-D fp16 tensor with unit column stride")
    m, n = x.shape
    if smooth_scale.dtype != torch.float32 or smooth_scale.numel() != n:
        raise ValueError("smooth_scale must be fp32 with N elements")
    q = out if out is not None else torch.empty((m, n), dtype=torch.int8, device=x.device)
    r = row_scale if row_scale is not None else torch.empty(m, dtype=torch.float32,
                                                            device=x.device)
    _lib.call("w8a8_smoothquant", _ptr(x), _ptr(smooth_scale.contiguous()), _ptr(q), _ptr(r),
              m, n, float(quant_max), x.stride(0), q.stride(0), _stream(x.device))
    return q, r


def moe_smoothquant(x, smooth_scale, topk_ids, quant_max: float = 127.0, dst_row=None,
                    rows: int | None = None, out=None, row_scale=None):
    """Per-expert smooth quantization of x [tokens, hidden].

    smooth_scale fp32 [experts, hidden]; topk_ids int32 [tokens, topk].
    Without dst_row the output is token-major [tokens*topk, hidden] (reference
    layout); with dst_row (int32 [tokens*topk]) pair i lands in row dst_row[i]
    of an output with `rows` rows (expert-sorted layout).
    """
    torch = _torch()
    _require_cuda(x, smooth_scale, topk_ids, dst_row)
    tokens, hidden = x.shape
    experts = smooth_scale.shape[0]
    topk = topk_ids.shape[1]
    nrows = rows if rows is not None else tokens * topk
    q = out if out is not None else torch.empty((nrows, hidden), dtype=torch.int8,
                                                device=x.device)
    r = row_scale if row_scale is not None else torch.empty(nrows, dtype=torch.float32,
                                                            device=x.device)
    _lib.call("w8a8_moe_smoothquant", _ptr(x.contiguous()), _ptr(smooth_scale.contiguous()),
              _ptr(topk_ids.contiguous()), _ptr(q), _ptr(r), tokens, hidden, topk, experts,
              float(quant_max), _ptr(dst_row), nrows, _stream(x.device))
    return q, r


def gemm_workspace_size(m: int, n: int, k: int, layout: int = LAYOUT_A_ROW_B_NK) -> int:
    return int(library().w8a8_gemm_workspace_size(m, n, k, layout))


def gemm(a, b, scale_a=None, scale_b=None, tensor_scale_a: float = 1.0,
         tensor_scale_b: float = 1.0, out_dtype=None, layout: int = LAYOUT_A_ROW_B_NK,
         out=None, workspace=None, m: int | None = None, n: int | None = None,
         k: int | None = None):
    """int8 GEMM with fused dequant.

    layout LAYOUT_A_ROW_B_NK: a int8 [M, K] (row stride lda), b int8 [N, K].
    layout LAYOUT_A_COL_B_KN: a int8 col-major (a is the [K, M] row-major
    tensor), b int8 [K, N] row-major: the reference sample's layout.
    out_dtype torch.int32 returns raw accumulators, torch.float16 the dequant.
    """
    torch = _torch()
    _require_cuda(a, b, scale_a, scale_b)
    out_dtype = out_dtype or torch.float16
    if layout == LAYOUT_A_ROW_B_NK:
        m = m or a.shape[0]
        k = k or a.shape[1]
        n = n or b.shape[0]
    else:
        k = k or a.shape[0]
        m = m or a.shape[1]
        n = n or b.shape[1]
    lda, ldb = a.stride(0), b.stride(0)
    c = out if out is not None else torch.empty((m, n), dtype=out_dtype, device=a.device)
    otype = OUT_I32 if c.dtype == torch.int32 else OUT_F16
    ws_bytes = gemm_workspace_size(m, n, k, layout)
    if workspace is None and ws_bytes:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=a.device)
    _lib.call("w8a8_gemm", m, n, k, _ptr(a), _ptr(b), _ptr(c), lda, ldb, c.stride(0),
              _ptr(scale_a), _ptr(scale_b), float(tensor_scale_a), float(tensor_scale_b), otype,
              layout, _ptr(workspace), workspace.numel() if workspace is not None else 0,
              _stream(a.device))
    return c


def fused_sq_gemm(x, smooth_scale, w, scale_w, out=None, q=None, row_scale=None):
    """SmoothQuant x [M, K] then C = dequant(q . w^T): returns (c fp16 [M, N], q, row_scale)."""
    torch = _torch()
    _require_cuda(x, smooth_scale, w, scale_w)
    m, k = x.shape
    n = w.shape[0]
    c = out if out is not None else torch.empty((m, n), dtype=torch.float16, device=x.device)
    q = q if q is not None else torch.empty((m, k), dtype=torch.int8, device=x.device)
    r = row_scale if row_scale is not None else torch.empty(m, dtype=torch.float32,
                                                            device=x.device)
    _lib.call("w8a8_fused_sq_gemm", _ptr(x), _ptr(smooth_scale), _ptr(w), _ptr(scale_w), _ptr(c),
              m, n, k, x.stride(0), w.stride(0), c.stride(0), _ptr(q), _ptr(r),
              _stream(x.device))
    return c, q, r


class PackedWeights:
    """int8 weights [n, k] packed into MFMA register order (w8a8_pack_weights).

    `data` is the packed uint8-sized device buffer; n and k are the logical
    weight shape.  Pack once at load time, then run gemm_packed /
    fused_sq_gemm_packed for every token batch.
    """

    def __init__(self, data, n: int, k: int):
        self.data = data
        self.n = int(n)
        self.k = int(k)

    @property
    def shape(self):
        return (self.n, self.k)


def pack_weights_size(n: int, k: int) -> int:
    return int(library().w8a8_pack_weights_size(n, k))


def pack_weights(w, out=None) -> PackedWeights:
    """Pack int8 weights w [N, K] (K-contiguous rows, any row stride)."""
    torch = _torch()
    _require_cuda(w)
    n, k = w.shape
    nbytes = pack_weights_size(n, k)
    buf = out if out is not None else torch.empty(nbytes, dtype=torch.int8, device=w.device)
    _lib.call("w8a8_pack_weights", _ptr(w), n, k, w.stride(0), _ptr(buf), buf.numel(),
              _stream(w.device))
    return PackedWeights(buf, n, k)


def gemm_packed(a, pw: PackedWeights, scale_a=None, scale_b=None, tensor_scale_a: float = 1.0,
                tensor_scale_b: float = 1.0, out_dtype=None, out=None):
    """gemm(a, w, ...) with w given as PackedWeights; a int8 [M, K] row-major."""
    torch = _torch()
    _require_cuda(a, pw.data, scale_a, scale_b)
    out_dtype = out_dtype or torch.float16
    m, k = a.shape
    if k != pw.k:
        raise ValueError(f"a has K={k}, packed weights K={pw.k}")
    c = out if out is not None else torch.empty((m, pw.n), dtype=out_dtype, device=a.device)
    otype = OUT_I32 if c.dtype == torch.int32 else OUT_F16
    _lib.call("w8a8_gemm_packed", m, pw.n, k, _ptr(a), _ptr(pw.data), _ptr(c), a.stride(0),
              c.stride(0), _ptr(scale_a), _ptr(scale_b), float(tensor_scale_a),
              float(tensor_scale_b), otype, _stream(a.device))
    return c


def fused_sq_gemm_packed(x, smooth_scale, pw: PackedWeights, scale_w, out=None, q=None,
                         row_scale=None):
    """fused_sq_gemm with PackedWeights: returns (c fp16 [M, N], q, row_scale)."""
    torch = _torch()
    _require_cuda(x, smooth_scale, pw.data, scale_w)
    m, k = x.shape
    if k != pw.k:
        raise ValueError(f"x has K={k}, packed weights K={pw.k}")
    c = out if out is not None else torch.empty((m, pw.n), dtype=torch.float16, device=x.device)
    q = q if q is not None else torch.empty((m, k), dtype=torch.int8, device=x.device)
    r = row_scale if row_scale is not None else torch.empty(m, dtype=torch.float32,
                                                            device=x.device)
    _lib.call("w8a8_fused_sq_gemm_packed", _ptr(x), _ptr(smooth_scale), _ptr(pw.data),
              _ptr(scale_w), _ptr(c), m, pw.n, k, x.stride(0), c.stride(0), _ptr(q), _ptr(r),
              _stream(x.device))
    return c, q, r
