"""Seeded, counter-based synthetic inputs for the W8A8 path.

Every element is a pure function of (seed, tensor id, flat index), so any slice
of any tensor can be regenerated independently (the CPU baseline and the GPU
run see identical inputs) and the values do not depend on chunking or on the
host.  The reference's own inputs are constant fills or time-seeded
(rocwmma_smoothquant.cpp:140-141, common.hpp:217-219), so this generator
defines what "identical seeded inputs" means for this path.

  h(seed, tid, i) = splitmix64 finalizer of (seed ^ tid << 56) + (i + 1) * 0x9E3779B97F4A7C15
  uniform         = (h >> 11) * 2^-53                              in [0, 1)
  normal          = Box-Muller on uniforms 2i, 2i+1 (double), then cast
  int8            = h % 255 - 127                                  in [-127, 127]
Tensor ids: X=1, s=2, outlier columns=3, A=4, B/W=5, sa=6, sb=7, logits=8,
expert s=9, W_down=10, sb_down=11.
"""
from __future__ import annotations

import concurrent.futures as _cf
import os

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

TID_X, TID_S, TID_OUTLIER, TID_A, TID_B, TID_SA, TID_SB = 1, 2, 3, 4, 5, 6, 7
TID_LOGITS, TID_EXPERT_S, TID_W_DOWN, TID_SB_DOWN = 8, 9, 10, 11
TID_RESIDUAL, TID_GAMMA = 12, 13  # RMSNorm residual stream and weight

_CHUNK = 1 << 22
# numpy releases the GIL inside its ufuncs, so chunks generate in parallel
# threads; every element is a function of its index alone, so the values do
# not depend on the thread count.
_THREADS = max(1, min(16, os.cpu_count() or 1))


def _parallel(starts, fn) -> None:
    starts = list(starts)
    if len(starts) <= 1 or _THREADS == 1:
        for s in starts:
            fn(s)
        return
    with _cf.ThreadPoolExecutor(max_workers=_THREADS) as ex:
        for _ in ex.map(fn, starts):
            pass


def config_seed(cfg: int) -> int:
    return 0x5EED0000 + cfg


def hash64(seed: int, tid: int, start: int, count: int) -> np.ndarray:
    """h(seed, tid, i) for i in [start, start + count) as uint64."""
    key = np.uint64((seed ^ (tid << 56)) & 0xFFFFFFFFFFFFFFFF)
    with np.errstate(over="ignore"):
        i = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        z = key + i * GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def _chunked(total: int, fn, dtype) -> np.ndarray:
    out = np.empty(total, dtype=dtype)

    def one(s):
        n = min(_CHUNK, total - s)
        out[s:s + n] = fn(s, n)

    _parallel(range(0, total, _CHUNK), one)
    return out


def uniform(seed: int, tid: int, shape, lo: float = 0.0, hi: float = 1.0,
            dtype=np.float32) -> np.ndarray:
    total = int(np.prod(shape))

    def fn(s, n):
        u = (hash64(seed, tid, s, n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
        return (lo + (hi - lo) * u).astype(dtype)

    return _chunked(total, fn, dtype).reshape(shape)


def normal(seed: int, tid: int, shape, dtype=np.float16) -> np.ndarray:
    total = int(np.prod(shape))

    def fn(s, n):
        h = hash64(seed, tid, 2 * s, 2 * n)
        u = (h >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
        u1 = 1.0 - u[0::2]  # (0, 1]
        u2 = u[1::2]
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        return z.astype(dtype)

    return _chunked(total, fn, dtype).reshape(shape)


def int8(seed: int, tid: int, shape) -> np.ndarray:
    total = int(np.prod(shape))

    def fn(s, n):
        return ((hash64(seed, tid, s, n) % np.uint64(255)).astype(np.int16) - 127).astype(np.int8)

    return _chunked(total, fn, np.int8).reshape(shape)


def outlier_columns(seed: int, k: int, frac: float = 0.005) -> np.ndarray:
    """round(frac * k) distinct column indices by seeded partial Fisher-Yates."""
    count = int(round(frac * k))
    perm = np.arange(k, dtype=np.int64)
    h = hash64(seed, TID_OUTLIER, 0, max(count, 1))
    for j in range(count):
        r = j + int(h[j] % np.uint64(k - j))
        perm[j], perm[r] = perm[r], perm[j]
    return np.sort(perm[:count])


def activations(seed: int, m: int, k: int, outlier_frac: float = 0.005,
                outlier_scale: float = 20.0) -> np.ndarray:
    """fp16 [m, k] N(0,1) with outlier columns scaled x20 before fp16 rounding."""
    cols = outlier_columns(seed, k, outlier_frac)
    out = np.empty((m, k), dtype=np.float16)
    rows_per = max(1, _CHUNK // max(k, 1))

    def one(r0):
        r1 = min(m, r0 + rows_per)
        h = hash64(seed, TID_X, 2 * r0 * k, 2 * (r1 - r0) * k)
        u = (h >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
        z = np.sqrt(-2.0 * np.log(1.0 - u[0::2])) * np.cos(2.0 * np.pi * u[1::2])
        z = z.reshape(r1 - r0, k)
        z[:, cols] *= outlier_scale
        out[r0:r1] = z.astype(np.float16)

    _parallel(range(0, m, rows_per), one)
    return out


def rmsnorm_inputs(seed: int, m: int, n: int):
    """RMSNorm inputs: x activation-like fp16 [m, n] (outlier columns included),
    residual N(0,1) fp16 [m, n], gamma fp32 U[0.5, 1.5] [n]."""
    x = activations(seed, m, n)
    res = normal(seed, TID_RESIDUAL, (m, n))
    gamma = uniform(seed, TID_GAMMA, (n,), 0.5, 1.5)
    return x, res, gamma
