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
  pack_weights / gemm_packed / fused_sq_gemm_packed
                   <- the pre-shuffled weights of flatmm (rocwmma_flatmm.cpp:12-16)
  grouped_gemm     <- grouped_gemm_kernel     (rocwmma_grouped_gemm.cpp:104-178)
  topk_softmax     <- kernel_topk_softmax     (rocwmma_topk_softmax.cpp:58-193)
  moe_sort         <- kernel_moe_histogram/prefix_sum/scatter (rocwmma_moe_sorting.cpp:53-125)
  moe_gemm, moe_silu_mul_quant, moe_combine, moe_ffn
                   <- the expert FFN chain (rocwmma_fused_moe.cpp:96-211), gate*up form
"""
from __future__ import annotations

from . import _lib
from ._lib import (  # noqa: F401
    ERROR_INVALID_VALUE,
    ERROR_NOT_SUPPORTED,
    FOLD_DIVIDE,
    FOLD_MULTIPLY,
    LAYOUT_A_COL_B_KN,
    LAYOUT_A_ROW_B_NK,
    OUT_F16,
    OUT_I32,
    STREAMK_WAIT_EXPIRED,
    W8A8Error,
)

__all__ = [
    "library", "version", "smoothquant", "moe_smoothquant", "gemm", "gemm_workspace_size",
    "gemm_streamk", "gemm_streamk_blocks", "gemm_streamk_status",
    "fused_sq_gemm", "W8A8Error", "PackedWeights", "pack_weights", "pack_weights_size",
    "gemm_packed", "gemm_packed_workspace_size", "fused_sq_gemm_packed", "grouped_gemm",
    "topk_softmax", "moe_sort", "moe_sort_workspace_size", "moe_gemm", "moe_gemm_workspace_size", "moe_silu_mul_quant",
    "moe_interleave_gate_up", "moe_gate_up_silu", "moe_gate_up_silu_workspace_size",
    "moe_combine", "moe_ffn", "add_rmsnorm_smoothquant", "rmsnorm", "add_rmsnorm",
    "quantize_weights",
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


def _rows2d(name, t, n=None):
    torch = _torch()
    if t.dim() != 2 or t.dtype != torch.float16 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D fp16 tensor with unit column stride")
    if n is not None and t.shape[1] != n:
        raise ValueError(f"{name} must have {n} columns")


def add_rmsnorm_smoothquant(x, gamma, smooth_scale=None, residual=None, eps: float = 1e-5,
                            quant_max: float = 127.0, x_out=None, want_y: bool = False,
                            y=None, q=None, row_scale=None):
    """RMSNorm of x (after `x + residual` when a residual is given) fused with
    the quantizer.

    Returns (x_out, y, q, row_scale); entries not requested are None.  x_out
    (= half(x + residual)) is produced when a residual is given; pass
    x_out=x (or =residual) to update in place.  y (the fp16 normalised row)
    is produced when want_y or y is given; q / row_scale when smooth_scale is
    given.  x, residual and x_out must share one row stride.
    """
    torch = _torch()
    _require_cuda(x, gamma, smooth_scale, residual, x_out, y, q, row_scale)
    _rows2d("x", x)
    m, n = x.shape
    if gamma.dtype != torch.float32 or gamma.numel() != n:
        raise ValueError("gamma must be fp32 with N elements")
    if residual is not None:
        _rows2d("residual", residual, n)
        if residual.shape != x.shape or residual.stride(0) != x.stride(0):
            raise ValueError("residual must match x in shape and row stride")
        if x_out is None:
            x_out = torch.empty_like(x)
        _rows2d("x_out", x_out, n)
        if x_out.shape != x.shape or x_out.stride(0) != x.stride(0):
            raise ValueError("x_out must match x in shape and row stride")
    elif x_out is not None:
        raise ValueError("x_out needs a residual")
    if want_y and y is None:
        y = torch.empty((m, n), dtype=torch.float16, device=x.device)
    if y is not None:
        _rows2d("y", y, n)
    if smooth_scale is not None:
        if smooth_scale.dtype != torch.float32 or smooth_scale.numel() != n:
            raise ValueError("smooth_scale must be fp32 with N elements")
        if q is None:
            q = torch.empty((m, n), dtype=torch.int8, device=x.device)
        if row_scale is None:
            row_scale = torch.empty(m, dtype=torch.float32, device=x.device)
        smooth_scale = smooth_scale.contiguous()
    else:
        q = row_scale = None
    _lib.call("w8a8_add_rmsnorm_smoothquant", _ptr(x), _ptr(residual), _ptr(gamma.contiguous()),
              _ptr(smooth_scale), _ptr(x_out), _ptr(y), _ptr(q), _ptr(row_scale), m, n,
              float(eps), float(quant_max), x.stride(0), y.stride(0) if y is not None else 0,
              q.stride(0) if q is not None else 0, _stream(x.device))
    return x_out, y, q, row_scale


def rmsnorm(x, gamma, eps: float = 1e-5):
    """fp16 RMSNorm y = half((x * rstd) * gamma) (kernel_rmsnorm2d_fwd's output)."""
    return add_rmsnorm_smoothquant(x, gamma, eps=eps, want_y=True)[1]


def add_rmsnorm(x, residual, gamma, eps: float = 1e-5):
    """(x_out, y) of kernel_add_rmsnorm2d_fwd: x_out = half(x + residual), y = RMSNorm(x_out)."""
    x_out, y, _, _ = add_rmsnorm_smoothquant(x, gamma, residual=residual, eps=eps, want_y=True)
    return x_out, y


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
    nrows = rows if rows is not None else (out.shape[0] if out is not None else tokens * topk)
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


def gemm_streamk(a, b, scale_a=None, scale_b=None, tensor_scale_a: float = 1.0,
                 tensor_scale_b: float = 1.0, out_dtype=None, blocks: int = 0, out=None,
                 workspace=None):
    """w8a8_gemm_streamk: the GEMM of gemm() (a int8 [M, K], b int8 [N, K]) with
    every tile's k-tiles cut into `blocks` equal ranges (0: the library picks,
    at most one per CU)."""
    torch = _torch()
    _require_cuda(a, b, scale_a, scale_b)
    out_dtype = out_dtype or torch.float16
    m, k = a.shape
    n = b.shape[0]
    c = out if out is not None else torch.empty((m, n), dtype=out_dtype, device=a.device)
    otype = OUT_I32 if c.dtype == torch.int32 else OUT_F16
    if workspace is None:
        ws_bytes = int(library().w8a8_gemm_streamk_workspace_size(m, n, k, blocks))
        workspace = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=a.device)
    _lib.call("w8a8_gemm_streamk", m, n, k, _ptr(a), _ptr(b), _ptr(c), a.stride(0), b.stride(0),
              c.stride(0), _ptr(scale_a), _ptr(scale_b), float(tensor_scale_a),
              float(tensor_scale_b), otype, blocks, _ptr(workspace), workspace.numel(),
              _stream(a.device))
    return c


def gemm_streamk_blocks(m: int, n: int, k: int, blocks: int = 0) -> int:
    """w8a8_gemm_streamk_blocks: the block count gemm_streamk launches."""
    return int(library().w8a8_gemm_streamk_blocks(m, n, k, blocks))


def gemm_streamk_status(clear: bool = True) -> int:
    """w8a8_gemm_streamk_status: the current device's sticky stream-K flags
    (STREAMK_WAIT_EXPIRED when a split tile's bounded wait gave up), read after
    a device-wide synchronisation; cleared when `clear`."""
    import ctypes

    flags = ctypes.c_uint32(0)
    _lib.call("w8a8_gemm_streamk_status", ctypes.byref(flags), 1 if clear else 0)
    return int(flags.value)


def fused_sq_gemm(x, smooth_scale, w, scale_w, out=None, q=None, row_scale=None,
                  workspace=None):
    """SmoothQuant x [M, K] then C = dequant(q . w^T): returns (c fp16 [M, N], q, row_scale).
    workspace: None (allocated here when the shape can use a K split, see
    gemm_workspace_size) or a device tensor; an empty tensor runs unsplit."""
    torch = _torch()
    _require_cuda(x, smooth_scale, w, scale_w)
    m, k = x.shape
    n = w.shape[0]
    c = out if out is not None else torch.empty((m, n), dtype=torch.float16, device=x.device)
    q = q if q is not None else torch.empty((m, k), dtype=torch.int8, device=x.device)
    r = row_scale if row_scale is not None else torch.empty(m, dtype=torch.float32,
                                                            device=x.device)
    if workspace is None:
        ws_bytes = gemm_workspace_size(m, n, k)
        if ws_bytes:
            workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=x.device)
    _lib.call("w8a8_fused_sq_gemm", _ptr(x), _ptr(smooth_scale), _ptr(w), _ptr(scale_w), _ptr(c),
              m, n, k, x.stride(0), w.stride(0), c.stride(0), _ptr(q), _ptr(r), _ptr(workspace),
              workspace.numel() if workspace is not None else 0, _stream(x.device))
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


def quantize_weights(w, smooth_scale=None, fold: int = FOLD_DIVIDE, packed: bool = True,
                     quant_max: float = 127.0, out=None, scale_w=None):
    """Offline weight preparation from fp16 w [N, K]: fold the smooth scale
    (FOLD_DIVIDE: w / s, the weight side of activations quantized as x * s;
    FOLD_MULTIPLY: w * s), quantize each output channel to int8 with an absmax
    scale, and pack (default) for gemm_packed / fused_sq_gemm_packed.

    Returns (PackedWeights or int8 [N, K] tensor, scale_w fp32 [N])."""
    torch = _torch()
    _require_cuda(w, smooth_scale, out, scale_w)
    if w.dim() != 2 or w.dtype != torch.float16 or w.stride(1) != 1:
        raise ValueError("w must be a 2-D fp16 tensor with unit column stride")
    n, k = w.shape
    if smooth_scale is not None:
        if smooth_scale.dtype != torch.float32 or smooth_scale.numel() != k:
            raise ValueError("smooth_scale must be fp32 with K elements")
        smooth_scale = smooth_scale.contiguous()
    sb = scale_w if scale_w is not None else torch.empty(n, dtype=torch.float32, device=w.device)
    if packed:
        buf = out if out is not None else torch.empty(pack_weights_size(n, k), dtype=torch.int8,
                                                      device=w.device)
        ldq, nbytes = 0, buf.numel()
    else:
        buf = out if out is not None else torch.empty((n, k), dtype=torch.int8, device=w.device)
        ldq, nbytes = buf.stride(0), (n - 1) * buf.stride(0) + k
    _lib.call("w8a8_quantize_weights", _ptr(w), n, k, w.stride(0), _ptr(smooth_scale), int(fold),
              float(quant_max), _ptr(buf), ldq, 1 if packed else 0, nbytes, _ptr(sb),
              _stream(w.device))
    return (PackedWeights(buf, n, k) if packed else buf), sb


def gemm_packed_workspace_size(m: int, n: int, k: int) -> int:
    """Bytes of split-K workspace the packed path can use for m x n x k (0: none)."""
    return int(library().w8a8_gemm_packed_workspace_size(m, n, k))


def _packed_workspace(workspace, m, n, k, device):
    return _workspace(workspace, lambda: gemm_packed_workspace_size(m, n, k), device)


def _workspace(workspace, size_fn, device):
    # "auto": allocate what the library asks for; None: run without (unsplit)
    if isinstance(workspace, str):
        if workspace != "auto":
            raise ValueError("workspace must be 'auto', None or a device tensor")
        size = size_fn()
        if size == 0:
            return None, 0
        workspace = _torch().empty(size, dtype=_torch().uint8, device=device)
    if workspace is None:
        return None, 0
    _require_cuda(workspace)
    return workspace, workspace.numel() * workspace.element_size()


def gemm_packed(a, pw: PackedWeights, scale_a=None, scale_b=None, tensor_scale_a: float = 1.0,
                tensor_scale_b: float = 1.0, out_dtype=None, out=None, workspace="auto"):
    """gemm(a, w, ...) with w given as PackedWeights; a int8 [M, K] row-major.
    workspace: 'auto' (allocated here when the shape uses one), None (no
    split-K), or a preallocated device tensor (see gemm_packed_workspace_size)."""
    torch = _torch()
    _require_cuda(a, pw.data, scale_a, scale_b)
    out_dtype = out_dtype or torch.float16
    m, k = a.shape
    if k != pw.k:
        raise ValueError(f"a has K={k}, packed weights K={pw.k}")
    c = out if out is not None else torch.empty((m, pw.n), dtype=out_dtype, device=a.device)
    otype = OUT_I32 if c.dtype == torch.int32 else OUT_F16
    ws, ws_bytes = _packed_workspace(workspace, m, pw.n, k, a.device)
    _lib.call("w8a8_gemm_packed", m, pw.n, k, _ptr(a), _ptr(pw.data), _ptr(c), a.stride(0),
              c.stride(0), _ptr(scale_a), _ptr(scale_b), float(tensor_scale_a),
              float(tensor_scale_b), otype, _ptr(ws), ws_bytes, _stream(a.device))
    return c


def fused_sq_gemm_packed(x, smooth_scale, pw: PackedWeights, scale_w, out=None, q=None,
                         row_scale=None, workspace="auto"):
    """fused_sq_gemm with PackedWeights: returns (c fp16 [M, N], q, row_scale).
    workspace as for gemm_packed."""
    torch = _torch()
    _require_cuda(x, smooth_scale, pw.data, scale_w)
    m, k = x.shape
    if k != pw.k:
        raise ValueError(f"x has K={k}, packed weights K={pw.k}")
    c = out if out is not None else torch.empty((m, pw.n), dtype=torch.float16, device=x.device)
    q = q if q is not None else torch.empty((m, k), dtype=torch.int8, device=x.device)
    r = row_scale if row_scale is not None else torch.empty(m, dtype=torch.float32,
                                                            device=x.device)
    ws, ws_bytes = _packed_workspace(workspace, m, pw.n, k, x.device)
    _lib.call("w8a8_fused_sq_gemm_packed", _ptr(x), _ptr(smooth_scale), _ptr(pw.data),
              _ptr(scale_w), _ptr(c), m, pw.n, k, x.stride(0), c.stride(0), _ptr(q), _ptr(r),
              _ptr(ws), ws_bytes, _stream(x.device))
    return c, q, r


def grouped_gemm(problems, out_dtype=None, outs=None):
    """One launch for several GEMMs.  problems: list of (a, b, scale_a, scale_b)
    with a int8 [M_g, K_g], b int8 [N_g, K_g] (scales may be None).  Returns the
    list of outputs (out_dtype torch.float16 or torch.int32)."""
    torch = _torch()
    out_dtype = out_dtype or torch.float16
    descs = (_lib.GroupDesc * len(problems))()
    results = []
    dev = None
    for i, (a, b, sa, sb) in enumerate(problems):
        _require_cuda(a, b, sa, sb)
        dev = a.device
        m, k = a.shape
        n = b.shape[0]
        c = outs[i] if outs is not None else torch.empty((m, n), dtype=out_dtype, device=dev)
        results.append(c)
        descs[i] = _lib.GroupDesc(a.data_ptr(), b.data_ptr(), c.data_ptr(), _ptr(sa), _ptr(sb),
                                  m, n, k, a.stride(0), b.stride(0), c.stride(0), 1.0, 1.0)
    otype = OUT_I32 if results[0].dtype == torch.int32 else OUT_F16
    ws_bytes = int(library().w8a8_grouped_gemm_workspace_size(len(problems)))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    # The descriptors are copied from this host array by an asynchronous copy
    # on the stream: keep the array alive until an event recorded after the
    # call has completed.  The workspace is freed through torch's caching
    # allocator, which orders its reuse on the stream.
    _lib.call("w8a8_grouped_gemm", descs, len(problems), otype, _ptr(ws), ws_bytes, _stream(dev))
    done = torch.cuda.Event()
    done.record(torch.cuda.current_stream(dev))
    _pending_descs[:] = [(e, d) for (e, d) in _pending_descs if not e.query()]
    _pending_descs.append((done, descs))
    return results


_pending_descs: list = []  # (event, host descriptor array) of grouped_gemm calls in flight


def topk_softmax(logits, topk: int, out=None):
    """logits fp32 or fp16 [T, E] -> (weights fp32 [T, topk], ids int32 [T, topk]).
    out: an optional (weights, ids) pair of contiguous tensors to write, so
    that a caller's loop (or a captured graph) allocates nothing."""
    torch = _torch()
    _require_cuda(logits)
    logits = logits.contiguous()
    t, e = logits.shape
    if out is not None:
        w, ids = out
        if (tuple(w.shape) != (t, topk) or w.dtype != torch.float32 or not w.is_contiguous()
                or tuple(ids.shape) != (t, topk) or ids.dtype != torch.int32
                or not ids.is_contiguous()):
            raise ValueError("topk_softmax: out must be contiguous (fp32 [T, topk], int32 [T, topk])")
        _require_cuda(w, ids)
    else:
        w = torch.empty((t, topk), dtype=torch.float32, device=logits.device)
        ids = torch.empty((t, topk), dtype=torch.int32, device=logits.device)
    _lib.call("w8a8_topk_softmax", _ptr(logits), 1 if logits.dtype == torch.float16 else 0,
              _ptr(w), _ptr(ids), t, e, topk, _stream(logits.device))
    return w, ids


def moe_sort_workspace_size(tokens: int, topk: int, experts: int) -> int:
    """Bytes of the optional moe_sort workspace (0: one workgroup suffices)."""
    return int(library().w8a8_moe_sort_workspace_size(tokens, topk, experts))


def moe_sort(topk_ids, experts: int, unit_size: int = 32, workspace="auto", out=None):
    """Stable expert sort of topk_ids int32 [T, k].  Returns a dict with
    count [E], start [E+1], padded [E], sorted_ids [capacity], dst_row [T*k].
    workspace: 'auto' (allocated here when T*k > 1024), None (one
    workgroup), or a device tensor of moe_sort_workspace_size bytes; the
    outputs are identical either way.  out: an optional dict of those five
    int32 tensors (contiguous, at least those sizes) to write instead of
    allocating them."""
    torch = _torch()
    _require_cuda(topk_ids)
    ids = topk_ids.contiguous()
    t, k = ids.shape
    cap = int(library().w8a8_moe_sort_capacity(t, k, experts, unit_size))
    d = ids.device
    sizes = dict(count=experts, start=experts + 1, padded=experts, sorted_ids=cap, dst_row=t * k)
    if out is not None:
        for name, size in sizes.items():
            v = out.get(name)
            if (v is None or v.dtype != torch.int32 or not v.is_contiguous()
                    or v.numel() < size):
                raise ValueError(f"moe_sort: out['{name}'] must be a contiguous int32 tensor of "
                                 f"at least {size} elements")
            _require_cuda(v)
    else:
        out = {name: torch.empty(size, dtype=torch.int32, device=d)
               for name, size in sizes.items()}
    ws, ws_bytes = _workspace(workspace, lambda: moe_sort_workspace_size(t, k, experts), d)
    _lib.call("w8a8_moe_sort", _ptr(ids), t, k, experts, unit_size, _ptr(out["count"]),
              _ptr(out["start"]), _ptr(out["padded"]), _ptr(out["sorted_ids"]), cap,
              _ptr(out["dst_row"]), _ptr(ws), ws_bytes, _stream(d))
    return out


def moe_gemm_workspace_size(experts: int, rows: int, n: int, k: int) -> int:
    """Bytes of the optional moe_gemm workspace (tail split along K)."""
    return int(library().w8a8_moe_gemm_workspace_size(experts, rows, n, k))


def moe_gemm(a, w, expert_start, expert_count, scale_a=None, scale_w=None, out_dtype=None,
             out=None, tensor_scale_a: float = 1.0, tensor_scale_b: float = 1.0,
             workspace="auto"):
    """Expert GEMM over expert-sorted rows: a int8 [rows, K], w int8 [E, N, K].
    workspace: 'auto' (allocated here), None (no tail split), or a
    preallocated device tensor of moe_gemm_workspace_size bytes; the result
    is bit-identical either way."""
    torch = _torch()
    _require_cuda(a, w, expert_start, expert_count, scale_a, scale_w)
    out_dtype = out_dtype or torch.float16
    rows, k = a.shape
    e, n, kw = w.shape
    if kw != k:
        raise ValueError(f"a has K={k}, weights K={kw}")
    c = out if out is not None else torch.empty((rows, n), dtype=out_dtype, device=a.device)
    otype = OUT_I32 if c.dtype == torch.int32 else OUT_F16
    ws, ws_bytes = _workspace(workspace, lambda: moe_gemm_workspace_size(e, rows, n, k), a.device)
    _lib.call("w8a8_moe_gemm", e, rows, n, k, _ptr(a), a.stride(0), _ptr(w), w.stride(1),
              w.stride(0), _ptr(c), c.stride(0), _ptr(scale_a), _ptr(scale_w),
              float(tensor_scale_a), float(tensor_scale_b), _ptr(expert_start),
              _ptr(expert_count), otype, _ptr(ws), ws_bytes, _stream(a.device))
    return c


def moe_silu_mul_quant(gate_up, expert_start, expert_count, smooth_scale=None,
                       quant_max: float = 127.0, q=None, row_scale=None):
    """gate_up fp16 [rows, 2*inter] -> (q int8 [rows, inter], row_scale fp32 [rows])."""
    torch = _torch()
    _require_cuda(gate_up, expert_start, expert_count, smooth_scale)
    rows, two_i = gate_up.shape
    inter = two_i // 2
    experts = expert_count.numel()
    q = q if q is not None else torch.empty((rows, inter), dtype=torch.int8, device=gate_up.device)
    r = row_scale if row_scale is not None else torch.empty(rows, dtype=torch.float32,
                                                            device=gate_up.device)
    _lib.call("w8a8_moe_silu_mul_quant", _ptr(gate_up), gate_up.stride(0), _ptr(smooth_scale),
              _ptr(expert_start), _ptr(expert_count), experts, rows, inter, _ptr(q), q.stride(0),
              _ptr(r), float(quant_max), _stream(gate_up.device))
    return q, r


def moe_interleave_gate_up(w_gate_up, scale_w=None):
    """gate_up weights int8 [E, 2*inter, K] (+ scales [E, 2*inter]) -> the row
    order moe_gate_up_silu reads (blocks of 16 gate rows then their 16 up rows)."""
    torch = _torch()
    e, two_i, k = w_gate_up.shape
    # the C ABI takes one row stride: rows of unit stride along K, experts
    # packed back to back at 2 * inter rows each
    if w_gate_up.stride(2) != 1 or w_gate_up.stride(0) != two_i * w_gate_up.stride(1):
        raise ValueError("moe_interleave_gate_up: w_gate_up must be [E, 2*inter, K] with unit "
                         "stride along K and experts 2*inter rows apart (call .contiguous())")
    if scale_w is not None and not scale_w.is_contiguous():
        raise ValueError("moe_interleave_gate_up: scale_w must be a contiguous [E, 2*inter]")
    _require_cuda(w_gate_up, scale_w)
    wo = torch.empty((e, two_i, k), dtype=torch.int8, device=w_gate_up.device)
    so = torch.empty((e, two_i), dtype=torch.float32, device=w_gate_up.device) \
        if scale_w is not None else None
    _lib.call("w8a8_moe_interleave_gate_up", _ptr(w_gate_up), _ptr(scale_w), e, two_i // 2, k,
              w_gate_up.stride(1), _ptr(wo), _ptr(so), _stream(w_gate_up.device))
    return wo, so


def moe_gate_up_silu_workspace_size(rows: int, inter: int) -> int:
    return int(library().w8a8_moe_gate_up_silu_workspace_size(rows, inter))


def moe_gate_up_silu(a, w_interleaved, expert_start, expert_count, scale_a=None,
                     scale_w_interleaved=None, smooth_scale=None, quant_max: float = 127.0,
                     q=None, row_scale=None, workspace=None, tensor_scale_a: float = 1.0,
                     tensor_scale_b: float = 1.0):
    """Gate_up expert GEMM with SiLU(gate)*up in its epilogue, then the
    requantization for the down GEMM: a int8 [rows, K] expert-sorted,
    w_interleaved from moe_interleave_gate_up -> (q int8 [rows, inter], row_scale)."""
    torch = _torch()
    rows, k = a.shape
    e, two_i, kw = w_interleaved.shape
    inter = two_i // 2
    # the C ABI reads the weights as a contiguous [E, 2*inter, K] (ldw = K)
    if kw != k or not w_interleaved.is_contiguous():
        raise ValueError(f"moe_gate_up_silu: w_interleaved must be a contiguous [E, 2*inter, K={k}]"
                         f" (got shape {tuple(w_interleaved.shape)}, "
                         f"strides {tuple(w_interleaved.stride())})")
    if a.stride(1) != 1:
        raise ValueError("moe_gate_up_silu: a must have unit stride along K")
    for name, t in (("scale_a", scale_a), ("scale_w_interleaved", scale_w_interleaved),
                    ("smooth_scale", smooth_scale)):
        if t is not None and not t.is_contiguous():
            raise ValueError(f"moe_gate_up_silu: {name} must be contiguous")
    _require_cuda(a, w_interleaved, expert_start, expert_count, scale_a, scale_w_interleaved,
                  smooth_scale)
    q = q if q is not None else torch.empty((rows, inter), dtype=torch.int8, device=a.device)
    r = row_scale if row_scale is not None else torch.empty(rows, dtype=torch.float32,
                                                            device=a.device)
    if workspace is None:
        workspace = torch.empty(moe_gate_up_silu_workspace_size(rows, inter), dtype=torch.uint8,
                                device=a.device)
    _lib.call("w8a8_moe_gate_up_silu", e, rows, inter, k, _ptr(a), a.stride(0),
              _ptr(w_interleaved), _ptr(scale_a), _ptr(scale_w_interleaved),
              float(tensor_scale_a), float(tensor_scale_b), _ptr(smooth_scale),
              _ptr(expert_start), _ptr(expert_count), _ptr(q), q.stride(0), _ptr(r),
              float(quant_max), _ptr(workspace), workspace.numel(), _stream(a.device))
    return q, r


def moe_combine(y, topk_weights, dst_row, out=None):
    """y fp16 [rows, N] (expert-sorted) -> out fp16 [T, N] = sum_k w * y[dst_row]."""
    torch = _torch()
    _require_cuda(y, topk_weights, dst_row)
    t, k = topk_weights.shape
    rows, n = y.shape
    o = out if out is not None else torch.empty((t, n), dtype=torch.float16, device=y.device)
    _lib.call("w8a8_moe_combine", _ptr(y), y.stride(0), rows, _ptr(topk_weights.contiguous()),
              _ptr(dst_row), t, k, n, _ptr(o), o.stride(0), _stream(y.device))
    return o


def moe_ffn(x, logits, smooth_scale, w_gate_up, sb_gate_up, w_down, sb_down, topk: int,
            smooth_scale_down=None, unit_size: int = 32, gate_up_interleaved=None):
    """Whole expert FFN on one GPU, nine launches, no host synchronization:
    top-k routing, stable expert sort, MoE SmoothQuant straight into the
    expert-sorted rows, gate_up expert GEMM, SiLU(gate)*up requantization,
    down expert GEMM, weighted combine.  Returns (out fp16 [T, H], parts).
    gate_up_interleaved: (w, scale) from moe_interleave_gate_up -- then the
    gate_up GEMM runs with the SiLU epilogue (moe_gate_up_silu) and
    parts["gate_up"] is None."""
    torch = _torch()
    t, h = x.shape
    e = w_gate_up.shape[0] if w_gate_up is not None else gate_up_interleaved[0].shape[0]
    w, ids = topk_softmax(logits, topk)
    srt = moe_sort(ids, e, unit_size)
    rows = srt["sorted_ids"].numel()
    qa = torch.empty((rows, h), dtype=torch.int8, device=x.device)
    ra = torch.empty(rows, dtype=torch.float32, device=x.device)
    moe_smoothquant(x, smooth_scale, ids, dst_row=srt["dst_row"], rows=rows, out=qa, row_scale=ra)
    ws = torch.empty(moe_gemm_workspace_size(e, rows, h, w_down.shape[2]), dtype=torch.uint8,
                     device=x.device)
    if gate_up_interleaved is not None:
        gu = None
        q2, r2 = moe_gate_up_silu(qa, gate_up_interleaved[0], srt["start"], srt["count"], ra,
                                  gate_up_interleaved[1], smooth_scale_down)
    else:
        gu = moe_gemm(qa, w_gate_up, srt["start"], srt["count"], ra, sb_gate_up, workspace=ws)
        q2, r2 = moe_silu_mul_quant(gu, srt["start"], srt["count"], smooth_scale_down)
    y = moe_gemm(q2, w_down, srt["start"], srt["count"], r2, sb_down, workspace=ws)
    out = moe_combine(y, w, srt["dst_row"])
    return out, dict(weights=w, ids=ids, sort=srt, qa=qa, ra=ra, gate_up=gu, q2=q2, r2=r2, y=y)
