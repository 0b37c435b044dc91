"""numpy bindings of the CPU oracle (oracle/liboracle.so) and of the reference
harness (oracle/_ref/libref.so).  Test infrastructure only: the product
library never loads either.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_DIR = ROOT / "oracle"
ORACLE_SO = ORACLE_DIR / "liboracle.so"
REF_SO = ORACLE_DIR / "_ref" / "libref.so"

_u32, _i32, _f32, _f64 = ctypes.c_uint32, ctypes.c_int, ctypes.c_float, ctypes.c_double
_p = ctypes.c_void_p

_ORACLE_SIGS = {
    "w8a8o_half_to_float": (_f32, [ctypes.c_uint16]),
    "w8a8o_float_to_half": (ctypes.c_uint16, [_f32]),
    "w8a8o_num_threads": (_i32, []),
    "w8a8o_smoothquant": (None, [_p, _p, _p, _p, _u32, _u32, _f32, _u32, _u32]),
    "w8a8o_moe_smoothquant": (None, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _f32, _p]),
    "w8a8o_gemm_i8_i32": (None, [_u32, _u32, _u32, _p, _p, _p, _u32, _u32, _u32, _i32, _u32,
                                 _u32]),
    "w8a8o_dequant_f16": (None, [_u32, _u32, _p, _u32, _p, _p, _f32, _f32, _p, _u32]),
    "w8a8o_topk_softmax": (None, [_p, _p, _p, _u32, _u32, _u32]),
    "w8a8o_moe_sort": (None, [_p, _u32, _u32, _u32, _u32, _p, _p, _p, _p, _p]),
    "w8a8o_silu_mul_quant": (None, [_p, _u32, _u32, _u32, _p, _f32, _p, _p, _u32]),
    "w8a8o_moe_combine": (None, [_p, _u32, _p, _p, _u32, _u32, _u32, _p, _u32]),
    "w8a8o_quantize_weights": (None, [_p, _p, _i32, _f32, _p, _p, _u32, _u32, _u32, _u32]),
    "w8a8o_rmsnorm_smoothquant": (None, [_p, _p, _p, _p, _p, _p, _p, _p, _u32, _u32, _f32, _f32,
                                         _u32, _u32, _u32]),
}

_REF_SIGS = {
    "ref_gemm_cpu_i8": (None, [_u32, _u32, _u32, _p, _p, _p, _u32, _u32, _u32, _i32]),
    "ref_compare_equal_f16": (_i32, [_p, _p, _u32, _f64, ctypes.POINTER(_f64)]),
    "ref_compare_equal_i32": (_i32, [_p, _p, _u32, _f64, ctypes.POINTER(_f64)]),
    "ref_kernel_smoothquant": (_i32, [_p, _p, _p, _p, _u32, _u32, _f32]),
    "ref_kernel_moe_smoothquant": (_i32, [_p, _p, _p, _p, _p, _u32, _u32, _u32, _u32, _f32]),
    "ref_kernel_topk_softmax": (_i32, [_p, _p, _p, _u32, _u32, _u32]),
    "ref_moe_sorting": (_i32, [_p, _u32, _u32, _u32, _u32, _p, _p, _p, _p, _p]),
    "ref_kernel_rmsnorm2d": (_i32, [_p, _p, _p, _u32, _u32, _u32, _u32, _f32]),
    "ref_kernel_add_rmsnorm2d": (_i32, [_p, _p, _p, _p, _p, _u32, _u32, _f32]),
}

_oracle = None
_ref = None


def build_oracle() -> None:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "oracle"], check=True)


def oracle() -> ctypes.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE_SO.exists():
            build_oracle()
        lib = ctypes.CDLL(str(ORACLE_SO))
        for name, (res, args) in _ORACLE_SIGS.items():
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        _oracle = lib
    return _oracle


def ref() -> ctypes.CDLL | None:
    """The reference-compiled harness, or None when it was not built."""
    global _ref
    if _ref is None:
        if not REF_SO.exists():
            return None
        try:  # share torch's HIP runtime (see optimized_rocwmma_samples_amd._lib)
            import torch  # noqa: F401
        except ImportError:
            pass
        lib = ctypes.CDLL(str(REF_SO))
        for name, (res, args) in _REF_SIGS.items():
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        _ref = lib
    return _ref


def _a(x: np.ndarray) -> int:
    assert x.flags.c_contiguous
    return x.ctypes.data


# ---------------------------------------------------------------- wrappers
def smoothquant(x: np.ndarray, s: np.ndarray, quant_max: float = 127.0):
    x = np.ascontiguousarray(x, dtype=np.float16)
    s = np.ascontiguousarray(s, dtype=np.float32)
    m, n = x.shape
    q = np.zeros((m, n), dtype=np.int8)
    r = np.zeros(m, dtype=np.float32)
    oracle().w8a8o_smoothquant(_a(x), _a(s), _a(q), _a(r), m, n, quant_max, n, n)
    return q, r


def moe_smoothquant(x, s, ids, quant_max=127.0, dst_row=None, rows=None, fill=0):
    x = np.ascontiguousarray(x, dtype=np.float16)
    s = np.ascontiguousarray(s, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    tokens, hidden = x.shape
    experts = s.shape[0]
    topk = ids.shape[1]
    nrows = rows if rows is not None else tokens * topk
    q = np.full((nrows, hidden), fill, dtype=np.int8)
    r = np.full(nrows, fill, dtype=np.float32)
    d = None if dst_row is None else np.ascontiguousarray(dst_row, dtype=np.int32)
    oracle().w8a8o_moe_smoothquant(_a(x), _a(s), _a(ids), _a(q), _a(r), tokens, hidden, topk,
                                   experts, quant_max, None if d is None else _a(d))
    return q, r


def gemm_i32(a: np.ndarray, b: np.ndarray, layout: int = 0, rows=None):
    """layout 0: a [M,K], b [N,K].  layout 1: a is [K,M] (col-major A), b [K,N]."""
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    if layout == 0:
        m, k = a.shape
        n = b.shape[0]
        lda, ldb = k, k
    else:
        k, m = a.shape
        n = b.shape[1]
        lda, ldb = m, n
    r0, r1 = (0, m) if rows is None else rows
    c = np.zeros((m, n), dtype=np.int32)
    oracle().w8a8o_gemm_i8_i32(m, n, k, _a(a), _a(b), _a(c), lda, ldb, n, layout, r0, r1)
    return c


def dequant_f16(acc: np.ndarray, sa=None, sb=None, tsa=1.0, tsb=1.0) -> np.ndarray:
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    m, n = acc.shape
    out = np.zeros((m, n), dtype=np.uint16)
    sa_ = None if sa is None else np.ascontiguousarray(sa, dtype=np.float32)
    sb_ = None if sb is None else np.ascontiguousarray(sb, dtype=np.float32)
    oracle().w8a8o_dequant_f16(m, n, _a(acc), n, None if sa_ is None else _a(sa_),
                               None if sb_ is None else _a(sb_), tsa, tsb, _a(out), n)
    return out.view(np.float16)


def ref_gemm_cpu_i8(a, b, layout=0):
    lib = ref()
    if lib is None:
        return None
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    if layout == 0:
        m, k = a.shape
        n = b.shape[0]
        lda, ldb = k, k
    else:
        k, m = a.shape
        n = b.shape[1]
        lda, ldb = m, n
    d = np.zeros((m, n), dtype=np.int32)
    lib.ref_gemm_cpu_i8(m, n, k, _a(a), _a(b), _a(d), lda, ldb, n, layout)
    return d


def ref_compare_equal(a: np.ndarray, b: np.ndarray, tol: float = 10.0):
    """The reference comparator compareEqual<T> (common.hpp:347-419)."""
    lib = ref()
    if lib is None:
        return None
    err = _f64(0.0)
    if a.dtype == np.float16:
        a = np.ascontiguousarray(a).view(np.uint16)
        b = np.ascontiguousarray(b).view(np.uint16)
        ok = lib.ref_compare_equal_f16(_a(a), _a(b), a.size, tol, ctypes.byref(err))
    else:
        a = np.ascontiguousarray(a, dtype=np.int32)
        b = np.ascontiguousarray(b, dtype=np.int32)
        ok = lib.ref_compare_equal_i32(_a(a), _a(b), a.size, tol, ctypes.byref(err))
    return bool(ok), err.value


def topk_softmax(logits: np.ndarray, topk: int):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    t, e = logits.shape
    w = np.zeros((t, topk), dtype=np.float32)
    ids = np.zeros((t, topk), dtype=np.int32)
    oracle().w8a8o_topk_softmax(_a(logits), _a(w), _a(ids), t, e, topk)
    return w, ids


def moe_sort(ids: np.ndarray, experts: int, unit_size: int):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    t, k = ids.shape
    count = np.zeros(experts, dtype=np.int32)
    start = np.zeros(experts + 1, dtype=np.int32)
    padded = np.zeros(experts, dtype=np.int32)
    sorted_ids = np.zeros(t * k + experts * unit_size, dtype=np.int32)
    dst = np.zeros(t * k, dtype=np.int32)
    oracle().w8a8o_moe_sort(_a(ids), t, k, experts, unit_size, _a(count), _a(start), _a(padded),
                            _a(sorted_ids), _a(dst))
    return count, start, padded, sorted_ids, dst


def silu_mul_quant(gate_up: np.ndarray, s2=None, quant_max=127.0):
    gu = np.ascontiguousarray(gate_up, dtype=np.float16)
    rows, two_i = gu.shape
    inter = two_i // 2
    q = np.zeros((rows, inter), dtype=np.int8)
    r = np.zeros(rows, dtype=np.float32)
    s2_ = None if s2 is None else np.ascontiguousarray(s2, dtype=np.float32)
    oracle().w8a8o_silu_mul_quant(_a(gu.view(np.uint16)), rows, inter, two_i,
                                  None if s2_ is None else _a(s2_), quant_max, _a(q), _a(r),
                                  inter)
    return q, r


def moe_combine(y: np.ndarray, weights: np.ndarray, dst_row: np.ndarray):
    y = np.ascontiguousarray(y, dtype=np.float16)
    w = np.ascontiguousarray(weights, dtype=np.float32)
    d = np.ascontiguousarray(dst_row, dtype=np.int32)
    t, k = w.shape
    n = y.shape[1]
    out = np.zeros((t, n), dtype=np.uint16)
    oracle().w8a8o_moe_combine(_a(y.view(np.uint16)), n, _a(w), _a(d), t, k, n, _a(out), n)
    return out.view(np.float16)


def rmsnorm_smoothquant(x: np.ndarray, gamma: np.ndarray, s=None, res=None, eps: float = 1e-5,
                        quant_max: float = 127.0):
    """(x_out, y, q, r) of the RMSNorm (+ residual) -> quantizer restatement;
    x_out is None without a residual, q and r are None without s."""
    x = np.ascontiguousarray(x, dtype=np.float16)
    g = np.ascontiguousarray(gamma, dtype=np.float32)
    m, n = x.shape
    rr = None if res is None else np.ascontiguousarray(res, dtype=np.float16)
    s_ = None if s is None else np.ascontiguousarray(s, dtype=np.float32)
    xo = None if rr is None else np.zeros((m, n), dtype=np.float16)
    y = np.zeros((m, n), dtype=np.float16)
    q = None if s_ is None else np.zeros((m, n), dtype=np.int8)
    r = None if s_ is None else np.zeros(m, dtype=np.float32)
    p = lambda a: None if a is None else _a(a)  # noqa: E731
    oracle().w8a8o_rmsnorm_smoothquant(_a(x), p(rr), _a(g), p(s_), p(xo), _a(y), p(q), p(r), m,
                                       n, eps, quant_max, n, n, n)
    return xo, y, q, r


def ref_rmsnorm2d_gpu(x, gamma, eps: float = 1e-5, residual=None):
    """Run the reference's own kernel_rmsnorm2d_fwd / kernel_add_rmsnorm2d_fwd
    (oracle/_ref) on device tensors; returns (x_out or None, y) as tensors."""
    import torch
    lib = ref()
    assert lib is not None, "oracle/_ref not built"
    m, n = x.shape
    y = torch.zeros_like(x)
    torch.cuda.synchronize()
    if residual is None:
        rc = lib.ref_kernel_rmsnorm2d(x.data_ptr(), gamma.data_ptr(), y.data_ptr(), m, n, n, n,
                                      eps)
        xo = None
    else:
        xo = torch.zeros_like(x)
        rc = lib.ref_kernel_add_rmsnorm2d(x.data_ptr(), residual.data_ptr(), gamma.data_ptr(),
                                          y.data_ptr(), xo.data_ptr(), m, n, eps)
    assert rc == 0, rc
    return xo, y


def quantize_weights(w: np.ndarray, s=None, divide: bool = True, quant_max: float = 127.0):
    """(q int8 [N, K], sb fp32 [N]) of the weight-quantization restatement."""
    w = np.ascontiguousarray(w, dtype=np.float16)
    n, k = w.shape
    s_ = None if s is None else np.ascontiguousarray(s, dtype=np.float32)
    q = np.zeros((n, k), dtype=np.int8)
    sb = np.zeros(n, dtype=np.float32)
    oracle().w8a8o_quantize_weights(_a(w.view(np.uint16)), None if s_ is None else _a(s_),
                                    1 if divide else 0, quant_max, _a(q), _a(sb), n, k, k, k)
    return q, sb
