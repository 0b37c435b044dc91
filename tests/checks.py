"""Comparison helpers shared by the GPU parity tests."""
from __future__ import annotations

import numpy as np


def dev(a, device):
    """numpy array -> torch tensor on `device` (contiguous copy)."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    return t.cpu().numpy()


def assert_i32_equal(got, exp):
    """Bit-exact int32 (the bar for accumulators)."""
    assert got.shape == exp.shape, (got.shape, exp.shape)
    if not np.array_equal(got, exp):
        bad = np.argwhere(got != exp)
        raise AssertionError(f"{len(bad)} int32 mismatches of {got.size}; first {bad[:4].tolist()}"
                             f" got {got[tuple(bad[0])]} exp {exp[tuple(bad[0])]}")


def assert_f16_bitexact(got, exp):
    """Bit-identical fp16, which implies the path's 1e-2 rel / 1e-3 abs bar; on a
    mismatch, report the bit-exact fraction and whether the bar still holds."""
    assert got.shape == exp.shape, (got.shape, exp.shape)
    if np.array_equal(got.view(np.uint16), exp.view(np.uint16)):
        return
    g, e = got.astype(np.float32), exp.astype(np.float32)
    fin = np.isfinite(e)
    within = bool(np.all(np.abs(g[fin] - e[fin]) <= 1e-3 + 1e-2 * np.abs(e[fin])))
    same = np.mean(got.view(np.uint16) == exp.view(np.uint16))
    raise AssertionError(f"fp16 bit-exact fraction {same:.6f}; within 1e-2 rel / 1e-3 abs: {within}")


def ulp_diff(a, b):
    """|a - b| in units in the last place of fp32 (same-sign finite values)."""
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)
