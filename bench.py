#!/usr/bin/env python3
"""Benchmark of the MI355X W8A8 SmoothQuant path (one GPU).

Headline (BASELINE.json metric "int8 TOPS (%MFMA peak) fused SQ+GEMM; SmoothQuant
GB/s (%HBM peak)", config 3): one step = SmoothQuant of the fp16 activations
followed by the int8 GEMM with fused per-token x per-channel dequant, for the
four Llama-3-8B projections at M=8192 tokens:
    qkv (K=4096, N=6144), o_proj (4096, 4096), gate_up (4096, 28672), down (14336, 4096)
value = total GEMM ops (2*M*N*K summed) / step time, in TOPS; inputs are
resident in HBM before timing starts.

Also reported: config 1 (standalone quantizer, X fp16 [2048, 4096]) in GB/s
with buffer sets rotated over >512 MB so the 256 MB MALL cannot serve repeats,
config 2 (W8A8 GEMM 4096^3 + dequant) in TOPS, and config 4 (decode: fused
SmoothQuant + packed-weight GEMM at M in {1, 16, 64} on the Llama-70B MLP
weights) in GB/s, and config 5 (Mixtral-shaped MoE FFN chain) in TOPS.
Per-kernel durations come from HIP events recorded on the stream the kernels
run on.

    python bench.py [--gpus 1] [--steps 10] [--warmup 3] [--m 8192] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_INT8_OPS = 5.0e15   # MI355X dense int8 MFMA, ops/s
PEAK_HBM_BPS = 8.0e12    # MI355X HBM3E, bytes/s

LLAMA3_8B = [("qkv", 4096, 6144), ("o_proj", 4096, 4096), ("gate_up", 4096, 28672),
             ("down", 14336, 4096)]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_projection(torch, dev, m, k, n):
    """cfg3 inputs of one projection from the seeded streams of
    optimized_rocwmma_samples_amd.datagen (seed 0x5EED0003; tensor ids X, s,
    B, sb), the same values the cfg3 parity tests check, copied to HBM."""
    from optimized_rocwmma_samples_amd import datagen as G

    seed = G.config_seed(3)
    x = torch.from_numpy(G.activations(seed, m, k)).to(dev)
    s = torch.from_numpy(G.uniform(seed, G.TID_S, (k,), 0.5, 2.0)).to(dev)
    w = torch.from_numpy(G.int8(seed, G.TID_B, (n, k))).to(dev)
    sb = torch.from_numpy(G.uniform(seed, G.TID_SB, (n,), 1e-3, 1e-2)).to(dev)
    q = torch.empty((m, k), dtype=torch.int8, device=dev)
    r = torch.empty(m, dtype=torch.float32, device=dev)
    c = torch.empty((m, n), dtype=torch.float16, device=dev)
    return dict(x=x, s=s, w=w, sb=sb, q=q, r=r, c=c, m=m, k=k, n=n)


def cpu_baseline(projs, rows: int):
    """Reference CPU path on a row sample of every projection: oracle SmoothQuant
    (port of rocwmma_smoothquant.cpp:74-121) + the reference's gemm_cpu_h
    (common.hpp:299-345, compiled from source into oracle/_ref) + dequant."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O

    use_ref = O.ref() is not None
    ops = 0.0
    t0 = time.perf_counter()
    for p in projs:
        x = p["x"][:rows].cpu().numpy()
        s = p["s"].cpu().numpy()
        w = p["w"].cpu().numpy()
        sb = p["sb"].cpu().numpy()
        t_start = time.perf_counter()
        q, r = O.smoothquant(x, s)
        acc = O.ref_gemm_cpu_i8(q, w) if use_ref else O.gemm_i32(q, w)
        O.dequant_f16(acc, r, sb)
        ops += 2.0 * rows * p["n"] * p["k"]
        log(f"cpu baseline {p['k']}x{p['n']} rows={rows}: {time.perf_counter() - t_start:.2f}s")
    dt = time.perf_counter() - t0
    threads = int(O.oracle().w8a8o_num_threads())
    return {
        "value": ops / dt / 1e12,
        "unit": "TOPS",
        "cores": threads,
        "kind": "reference" if use_ref else "port",
        "sample": (f"{rows} of 8192 rows of each Llama-3-8B projection (qkv, o_proj, gate_up, "
                   f"down): SmoothQuant (oracle port) + gemm_cpu_h "
                   f"({'reference common.hpp' if use_ref else 'oracle port'}) + dequant; "
                   f"{ops / 1e9:.1f} GOP in {dt:.1f} s"),
    }


def _oracle_libs():
    """The CPU checkers (oracle port; the reference's gemm_cpu_h when
    oracle/_ref was built) and the OpenMP thread count they run on."""
    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib as O

    return O, O.ref() is not None, int(O.oracle().w8a8o_num_threads())


def cpu_baseline_quantizer(x, s, nbytes, budget_s=3.0):
    """cfg1 on the host: the oracle quantizer (port of
    rocwmma_smoothquant.cpp:74-121) over the whole cfg1 problem, repeated for
    about budget_s seconds; GB/s over the same algorithmic bytes as the GPU
    launch."""
    O, _, threads = _oracle_libs()
    O.smoothquant(x, s)  # first-touch of the outputs, thread pool start
    reps, t0 = 0, time.perf_counter()
    while True:
        O.smoothquant(x, s)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            break
    return {"value": nbytes * reps / dt / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the whole cfg1 problem (X fp16 [{x.shape[0]}, {x.shape[1]}]), {reps} "
                      f"runs of the oracle quantizer in {dt:.1f} s"}


def cpu_baseline_decode(layers, m=16):
    """cfg4 on the host at M = 16 (the reference's gemm_cpu_h parallelizes over
    rows: one thread per row): SmoothQuant of the activations (oracle port),
    gemm_cpu_h over the whole weight matrix, dequant, for each Llama-70B MLP
    weight; GB/s over the same algorithmic bytes as the GPU layers."""
    O, use_ref, threads = _oracle_libs()
    nbytes, t0 = 0, time.perf_counter()
    for x, s, w, sb in layers:
        n, k = w.shape
        q, r = O.smoothquant(x[:m], s)
        acc = O.ref_gemm_cpu_i8(q, w) if use_ref else O.gemm_i32(q, w)
        O.dequant_f16(acc, r, sb)
        nbytes += n * k + 4 * n + 2 * m * k + 4 * k + 2 * (m * k + 4 * m) + 2 * m * n
    dt = time.perf_counter() - t0
    return {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": min(threads, m),
            "kind": "reference" if use_ref else "port",
            "sample": f"M = {m}, both weights W1 [28672, 8192] and W2 [8192, 28672] whole: "
                      f"SmoothQuant (oracle port) + gemm_cpu_h "
                      f"({'reference common.hpp' if use_ref else 'oracle port'}) + dequant, "
                      f"{nbytes / 1e9:.2f} GB of layer bytes in {dt:.1f} s"}


def cpu_baseline_moe(x, logits, s, wgu, sgu, wd, sd, topk, rows_per_expert=16):
    """cfg5 on the host: routing, sort and the MoE quantizer over all 4096
    tokens (oracle port), then for the first `rows_per_expert` sorted rows of
    every expert the gate_up GEMM (gemm_cpu_h), dequant, SiLU(gate)*up
    requant (oracle), down GEMM and dequant; TOPS over those rows' GEMM ops."""
    O, use_ref, threads = _oracle_libs()
    gemm = O.ref_gemm_cpu_i8 if use_ref else O.gemm_i32
    e = s.shape[0]
    t0 = time.perf_counter()
    w, ids = O.topk_softmax(logits, topk)
    count, start, padded, sorted_ids, dst = O.moe_sort(ids, e, 32)
    qa, ra = O.moe_smoothquant(x, s, ids, dst_row=dst, rows=sorted_ids.size)
    ops = 0.0
    for xe in range(e):
        r0 = int(start[xe])
        r1 = r0 + min(rows_per_expert, int(count[xe]))
        if r1 == r0:
            continue
        gu = O.dequant_f16(gemm(qa[r0:r1], wgu[xe]), ra[r0:r1], sgu[xe])
        q2, r2 = O.silu_mul_quant(gu)
        O.dequant_f16(gemm(q2, wd[xe]), r2, sd[xe])
        ops += 2.0 * (r1 - r0) * (wgu.shape[1] * wgu.shape[2] + wd.shape[1] * wd.shape[2])
    dt = time.perf_counter() - t0
    return {"value": ops / dt / 1e12, "unit": "TOPS", "cores": min(threads, rows_per_expert),
            "kind": "reference" if use_ref else "port",
            "sample": f"routing + sort + MoE quantizer over all {x.shape[0]} tokens, then "
                      f"{rows_per_expert} sorted rows of each of the {e} experts through gate_up "
                      f"gemm_cpu_h ({'reference common.hpp' if use_ref else 'oracle port'}) + "
                      f"SiLU requant + down: {ops / 1e9:.1f} GOP in {dt:.1f} s"}


def graph_us(torch, calls, repeat=1):
    """Per-call GPU time of `calls` (a list of closures that enqueue work on
    torch's current stream): captured once into a HIP graph on a side stream,
    replayed once to warm up, then one replay timed between two events.  The
    host's launch cost does not enter: short kernels are timed back to back,
    as the reference samples time their launch loops (README.md:1568-1569)."""
    # the side stream does not wait for the default stream by itself: without
    # this, the warm-up calls could read inputs still being generated, and
    # write outputs into memory that a pending kernel still reads
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        for c in calls[:3]:
            c()  # one-time setup (LDS limits) stays out of the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        for _ in range(repeat):
            for c in calls:
                c()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(st):
        e0.record()
        g.replay()
        e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (len(calls) * repeat)


def quantizer_sets(torch, dev, gen, m, n, nsets):
    sets = []
    for _ in range(nsets):
        x = torch.randn((m, n), generator=gen, device=dev).to(torch.float16)
        s = torch.rand(n, generator=gen, device=dev) * 1.5 + 0.5
        sets.append((x, s, torch.empty((m, n), dtype=torch.int8, device=dev),
                     torch.empty(m, dtype=torch.float32, device=dev)))
    return sets


def bench_quantizer(torch, w8a8, dev, gen, iters=48, cpu=True):
    """Config 1: X fp16 [2048, 4096].  Cold: 24 buffer sets (600 MB, over the
    256 MB MALL) used in turn, so every launch reads HBM; warm: one set
    relaunched, as the reference measures (inputs MALL-resident).  cpu: the
    oracle quantizer timed on the host over the first set."""
    m, n = 2048, 4096
    sets = quantizer_sets(torch, dev, gen, m, n, 24)
    calls = [(lambda b=sets[i % len(sets)]: w8a8.smoothquant(b[0], b[1], out=b[2], row_scale=b[3]))
             for i in range(iters)]
    cold = graph_us(torch, calls)
    warm = graph_us(torch, calls[:1], repeat=iters)
    nbytes = 2 * m * n + 4 * n + m * n + 4 * m  # rocwmma_smoothquant.cpp:157-158
    return {"workload": "cfg1 X fp16 [2048,4096] -> int8 (graph-replayed launches)",
            "bytes_per_launch": nbytes,
            "us_per_launch": cold, "GBps": nbytes / (cold * 1e-6) / 1e9,
            "frac_hbm": nbytes / (cold * 1e-6) / PEAK_HBM_BPS,
            "warm_us_per_launch": warm, "warm_GBps": nbytes / (warm * 1e-6) / 1e9,
            "note": "cold = 24 rotating buffer sets (every launch reads HBM); warm = one set, "
                    "MALL-resident like the reference's repeated launches",
            "cpu_baseline": (cpu_baseline_quantizer(sets[0][0].cpu().numpy(),
                                                    sets[0][1].cpu().numpy(), nbytes)
                             if cpu else None)}


def bench_quantizer_sweep(torch, w8a8, dev, gen):
    """Quantizer rate as the call grows (N = 4096 and the cfg3 widths), cold."""
    out = []
    for m, n in [(2048, 4096), (8192, 4096), (32768, 4096), (131072, 4096), (8192, 14336)]:
        per = 3 * m * n
        nsets = max(1, min(24, (600 << 20) // per + 1))
        sets = quantizer_sets(torch, dev, gen, m, n, nsets)
        iters = max(8, 2 * nsets)
        calls = [(lambda b=sets[i % nsets]: w8a8.smoothquant(b[0], b[1], out=b[2],
                                                             row_scale=b[3]))
                 for i in range(iters)]
        us = graph_us(torch, calls)
        nbytes = 3 * m * n + 4 * n + 4 * m
        out.append({"M": m, "N": n, "us": us, "GBps": nbytes / (us * 1e-6) / 1e9,
                    "frac_hbm": nbytes / (us * 1e-6) / PEAK_HBM_BPS})
        del sets
    return out


def bench_rmsnorm_sq(torch, w8a8, dev, gen, iters=12):
    """Add+RMSNorm fused with the quantizer at the cfg3 token count: the
    residual stream x + res -> x_out and the int8 A operand of the next GEMM
    (q, row scale), M = 8192 rows of hidden 4096.  Three buffer sets (700 MB)
    used in turn, so every launch reads HBM; the unfused chain (Add+RMSNorm
    writing fp16 y, then the quantizer reading it) is timed the same way."""
    m, n = 8192, 4096
    sets = []
    for _ in range(3):
        x = torch.randn((m, n), generator=gen, device=dev).to(torch.float16)
        r = torch.randn((m, n), generator=gen, device=dev).to(torch.float16)
        sets.append((x, r, torch.empty_like(x), torch.empty((m, n), dtype=torch.int8, device=dev),
                     torch.empty(m, dtype=torch.float32, device=dev)))
    g = torch.rand(n, generator=gen, device=dev) + 0.5
    s = torch.rand(n, generator=gen, device=dev) * 1.5 + 0.5
    y = torch.empty((m, n), dtype=torch.float16, device=dev)

    def fused(b):
        w8a8.add_rmsnorm_smoothquant(b[0], g, s, residual=b[1], x_out=b[2], q=b[3], row_scale=b[4])

    def chain(b):
        w8a8.add_rmsnorm_smoothquant(b[0], g, residual=b[1], x_out=b[2], y=y)
        w8a8.smoothquant(y, s, out=b[3], row_scale=b[4])

    t_fused = graph_us(torch, [(lambda b=sets[i % 3]: fused(b)) for i in range(iters)])
    t_chain = graph_us(torch, [(lambda b=sets[i % 3]: chain(b)) for i in range(iters)])
    nbytes = 2 * m * n * 3 + m * n + 4 * m + 8 * n  # x, res in; x_out, q, r out; gamma, s
    return {"workload": "Add+RMSNorm -> SmoothQuant, M=8192 hidden=4096 (Llama-3-8B layer input)",
            "bytes_per_launch": nbytes, "us_per_launch": t_fused,
            "GBps": nbytes / (t_fused * 1e-6) / 1e9,
            "frac_hbm": nbytes / (t_fused * 1e-6) / PEAK_HBM_BPS,
            "unfused_chain_us": t_chain, "speedup_vs_unfused": t_chain / t_fused}


def bench_gemm_4096(torch, w8a8, dev, gen, iters=20):
    m = n = k = 4096
    a = torch.randint(-127, 128, (m, k), generator=gen, device=dev, dtype=torch.int8)
    b = torch.randint(-127, 128, (n, k), generator=gen, device=dev, dtype=torch.int8)
    sa = torch.rand(m, generator=gen, device=dev) * 9e-3 + 1e-3
    sb = torch.rand(n, generator=gen, device=dev) * 9e-3 + 1e-3
    c = torch.empty((m, n), dtype=torch.float16, device=dev)
    for _ in range(3):
        w8a8.gemm(a, b, sa, sb, out=c)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        w8a8.gemm(a, b, sa, sb, out=c)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / iters * 1e3
    tops = 2.0 * m * n * k / (us * 1e-6) / 1e12
    return {"workload": "cfg2 4096^3 int8 GEMM + fp16 dequant", "us_per_launch": us,
            "TOPS": tops, "frac_mfma": tops * 1e12 / PEAK_INT8_OPS}


def bench_decode(torch, w8a8, dev, gen, iters=20, cpu=True):
    """Config 4: fused SmoothQuant + packed-weight decode GEMM, Llama-70B MLP
    weights W1 [28672, 8192] and W2 [8192, 28672] at M in {1, 16, 64}.  Two
    copies of each weight (2 x 235 MB per shape, over the 256 MB MALL) are
    used in turn, so a launch does not find its weights in MALL."""
    shapes = [(28672, 8192), (8192, 28672)]
    weights, host_w = {}, {}
    for n, k in shapes:
        copies = []
        for c in range(2):
            w = torch.randint(-127, 128, (n, k), generator=gen, device=dev, dtype=torch.int8)
            copies.append(w8a8.pack_weights(w))
            if cpu and c == 0:
                host_w[(n, k)] = w.cpu().numpy()
            del w
        sb = torch.rand(n, generator=gen, device=dev) * 9e-3 + 1e-3
        weights[(n, k)] = (copies, sb)
    cpu_layers = []
    results = []
    for m in (1, 16, 64):
        bufs = {}
        for n, k in shapes:
            x = torch.randn((m, k), generator=gen, device=dev).to(torch.float16)
            s = torch.rand(k, generator=gen, device=dev) * 1.5 + 0.5
            bufs[(n, k)] = (x, s, torch.empty((m, k), dtype=torch.int8, device=dev),
                            torch.empty(m, dtype=torch.float32, device=dev),
                            torch.empty((m, n), dtype=torch.float16, device=dev))
        for (n, k) in shapes:
            x, s, q, r, out = bufs[(n, k)]
            copies, sb = weights[(n, k)]
            if cpu and m == 16:
                cpu_layers.append((x.cpu().numpy(), s.cpu().numpy(), host_w[(n, k)],
                                   sb.cpu().numpy()))
            # split-K workspace (M = 64 takes one), allocated once
            wsz = w8a8.gemm_packed_workspace_size(m, n, k)
            ws = torch.empty(wsz, dtype=torch.uint8, device=dev) if wsz else None
            # the two copies alternate: each launch streams its weights from HBM
            calls = [(lambda c=copies[i % 2]: w8a8.fused_sq_gemm_packed(
                x, s, c, sb, out=out, q=q, row_scale=r, workspace=ws)) for i in range(iters)]
            us = graph_us(torch, calls)
            # algorithmic HBM bytes of the layer: weights once, activations
            # fp16 in, int8 + row scale round trip, scales, fp16 out
            nbytes = n * k + 4 * n + 2 * m * k + 4 * k + 2 * (m * k + 4 * m) + 2 * m * n
            results.append({"M": m, "N": n, "K": k, "us_per_layer": us,
                            "workspace_bytes": wsz,
                            "GBps": nbytes / (us * 1e-6) / 1e9,
                            "frac_hbm": nbytes / (us * 1e-6) / PEAK_HBM_BPS,
                            "TOPS": 2.0 * m * n * k / (us * 1e-6) / 1e12})
    return {"workload": "cfg4 decode: fused SmoothQuant + packed-weight GEMM, graph-replayed "
                        "(two weight copies per shape alternate: MALL-cold)", "layers": results,
            "cpu_baseline": cpu_baseline_decode(cpu_layers) if cpu else None}


TRAFFIC_PROFILE = ROOT / "profiles" / "gemm_i8_persist_and_tile_kernels__cfg3_llama3_8b_and_cfg2.md"
TRAFFIC_SECTION = "## HBM-side traffic of the cfg3 projections"


def projection_kernel(p, cus):
    """Which 256 x 256 kernel the library runs for an fp16 projection GEMM:
    the persistent kernel when there are at least two tiles per CU and at
    most 32 k-tiles of 128 (persist_pays, csrc/gemm_i8.hip), otherwise the
    one-tile-per-block kernel."""
    tiles = -(-p["m"] // 256) * -(-p["n"] // 256)
    return "persist" if tiles >= 2 * cus and -(-p["k"] // 128) <= 32 else "tile"


def profiled_traffic(projs, cus):
    """HBM-side bytes per launch of the projection GEMMs, averaged like
    `achieved`, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    of a bench run without the extras (scaled by the calibration copy).  The
    persistent kernel launches one block per CU for every projection it runs,
    so its launches share one (kernel, grid) row; where the profile also
    lists that kernel's dispatches by position in the step's launch order
    (`pos=<i>/<n>` lines, one per persistent projection), each projection
    gets its own, else the row's average.  Tile-kernel rows are keyed by
    their grid.  Returns (average, per projection, per-projection persistent
    entries by launch order?); None, None, False when the profile does not
    cover these launches."""
    import re
    if not TRAFFIC_PROFILE.exists():
        return None, None, False
    table, pos, on = {}, {}, False
    for line in TRAFFIC_PROFILE.read_text().splitlines():
        if line.startswith("## "):
            on = line.startswith(TRAFFIC_SECTION)
            continue
        if not on:
            continue
        mp = re.match(r"traffic \S*gemm_i8_persist_kernel<\S*Cfg<256,256,\S* grid=(\d+) "
                      r"pos=(\d+)/(\d+) .* bytes=(\d+)", line)
        if mp:
            pos[(int(mp.group(1)), int(mp.group(2)), int(mp.group(3)))] = int(mp.group(4))
            continue
        mt = re.match(r"traffic \S*gemm_i8_(tile|persist)_kernel<\S*Cfg<256,256,\S* grid=(\d+) .* bytes=(\d+)",
                      line)
        if mt:
            table[(mt.group(1), int(mt.group(2)))] = int(mt.group(3))
    kinds = [projection_kernel(p, cus) for p in projs]
    npersist = kinds.count("persist")
    by_order = npersist > 1 and all((cus * 512, i, npersist) in pos for i in range(npersist))
    per, ip = [], 0
    for p, kind in zip(projs, kinds):
        grid = cus * 512 if kind == "persist" else -(-p["m"] // 256) * -(-p["n"] // 256) * 512
        if (kind, grid) not in table:
            return None, None, False
        if kind == "persist" and by_order:
            per.append(pos[(grid, ip, npersist)])
            ip += 1
        else:
            per.append(table[(kind, grid)])
    return sum(per) / len(per), per, by_order


def bench_cfg3_smaller_m(torch, w8a8, dev, base, steps=10, sets=3):
    """Config 3 at its smaller token counts (M = 512, 2048): SmoothQuant +
    GEMM over the four Llama-3-8B projections, as in the headline step, with
    the dense GEMM's K-split workspace preallocated (the launches whose tiles
    fill at most half of the CUs use it).  Inputs are the first M rows of the
    headline's (datagen) activations; `sets` copies of its weights are used in
    turn so each step streams its weights from HBM (3 x 216 MB).  A step is 8
    launches of 3-70 us, so launching them one by one from Python costs about
    as much host time as the GPU spends: the steps are timed replayed from a
    captured HIP graph (`TOPS`, GPU throughput; one replay's outputs are
    checked bitwise against the eager step) and launched eagerly
    (`eager_TOPS`)."""
    def sub(p, m, copy):
        return dict(x=p["x"][:m], s=p["s"], w=p["w"].clone() if copy else p["w"], sb=p["sb"],
                    q=torch.empty((m, p["k"]), dtype=torch.int8, device=dev),
                    r=torch.empty(m, dtype=torch.float32, device=dev),
                    c=torch.empty((m, p["n"]), dtype=torch.float16, device=dev),
                    m=m, k=p["k"], n=p["n"])

    out = []
    for m in (512, 2048):
        projs = [[sub(p, m, i > 0) for p in base] for i in range(sets)]
        ws_bytes = max(w8a8.gemm_workspace_size(m, n, k) for (_, k, n) in LLAMA3_8B)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
        ops = sum(2.0 * m * n * k for (_, k, n) in LLAMA3_8B)

        def step(i, ev=None):
            for j, p in enumerate(projs[i % sets]):
                if ev is not None:
                    ev[j].record()
                w8a8.smoothquant(p["x"], p["s"], out=p["q"], row_scale=p["r"])
                w8a8.gemm(p["q"], p["w"], p["r"], p["sb"], out=p["c"], workspace=ws)
            if ev is not None:
                ev[len(projs[0])].record()

        for i in range(3):
            step(i)
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for i in range(steps):
            step(i)
        t1.record()
        torch.cuda.synchronize()
        eager_ms = t0.elapsed_time(t1) / steps
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(LLAMA3_8B) + 1)]
               for _ in range(steps)]
        for i in range(steps):
            step(i, evs[i])
        torch.cuda.synchronize()
        per = {name: sum(e[j].elapsed_time(e[j + 1]) for e in evs) / steps * 1e3
               for j, (name, _, _) in enumerate(LLAMA3_8B)}
        # the same steps replayed from a graph, then the last one's outputs
        # against an eager run of that step
        ms = graph_us(torch, [(lambda i=i: step(i)) for i in range(steps)]) / 1e3
        last = projs[(steps - 1) % sets]
        replayed = [p["c"].clone() for p in last]
        step(steps - 1)
        torch.cuda.synchronize()
        same = all(torch.equal(a.view(torch.int16), p["c"].view(torch.int16))
                   for a, p in zip(replayed, last))
        out.append({"M": m, "ms_per_step": ms, "TOPS": ops / (ms * 1e-3) / 1e12,
                    "frac_mfma": ops / (ms * 1e-3) / PEAK_INT8_OPS,
                    "graph_matches_eager": same,
                    "eager_ms_per_step": eager_ms,
                    "eager_TOPS": ops / (eager_ms * 1e-3) / 1e12,
                    "fused_us_per_projection": per, "workspace_bytes": ws_bytes})
        del projs, ws
    return out


def capture_graph(torch, calls, repeat=1):
    """Capture `calls` (closures enqueuing work on torch's current stream),
    `repeat` times over, into a HIP graph on a side stream after one eager
    pass of them there (one-time setup stays out of the capture).  Returns
    (graph, stream)."""
    torch.cuda.synchronize()
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        for c in calls:
            c()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        for _ in range(repeat):
            for c in calls:
                c()
    g.replay()
    torch.cuda.synchronize()
    return g, st


def replay_us(torch, g, st):
    """GPU time of one replay of g, between two events on its stream."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(st):
        e0.record()
        g.replay()
        e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3


def bench_moe(torch, w8a8, dev, gen, iters=10, rounds=6, cpu=True):
    """Config 5: Mixtral-8x7B-shaped MoE FFN, 4096 tokens, hidden 4096, ffn
    14336, 8 experts, top-2.  One layer = routing, sort, MoE SmoothQuant into
    expert-sorted rows, gate_up expert GEMM with the SiLU(gate)*up epilogue
    and the requantization (weights interleaved once beforehand), down expert
    GEMM, combine; ops = 2 * 8192 rows * (28672*4096 + 4096*14336).  The same
    layer with the gate_up GEMM and the SiLU requantization as two launches
    is the unfused form.
    Every buffer (routing and sort outputs included) is allocated once, and
    the layers are replayed from captured HIP graphs (`iters` layers per
    graph), so no host-side work or allocation can enter the timed region:
    the fused and unfused graphs alternate for `rounds` replays each after
    0.3 s of untimed layers (the clocks settle under this load), and the
    layer time is the mean over the replays.  Each stage is also timed alone,
    `iters` launches of it per graph (`stage_us`); the last fused replay's
    output is compared bitwise with an eager layer's."""
    t, h, inter, e, k = 4096, 4096, 14336, 8, 2
    x = torch.randn((t, h), generator=gen, device=dev)
    cols = torch.randperm(h, generator=gen, device=dev)[: round(0.005 * h)]
    x[:, cols] *= 20.0
    x = x.to(torch.float16)
    logits = torch.randn((t, e), generator=gen, device=dev)
    s = torch.rand((e, h), generator=gen, device=dev) * 1.5 + 0.5
    wgu = torch.randint(-127, 128, (e, 2 * inter, h), generator=gen, device=dev, dtype=torch.int8)
    sgu = torch.rand((e, 2 * inter), generator=gen, device=dev) * 9e-3 + 1e-3
    wgu_il, sgu_il = w8a8.moe_interleave_gate_up(wgu, sgu)
    wd = torch.randint(-127, 128, (e, h, inter), generator=gen, device=dev, dtype=torch.int8)
    sd = torch.rand((e, h), generator=gen, device=dev) * 9e-3 + 1e-3
    cap = int(w8a8.library().w8a8_moe_sort_capacity(t, k, e, 32))
    rw = torch.empty((t, k), dtype=torch.float32, device=dev)
    rid = torch.empty((t, k), dtype=torch.int32, device=dev)
    srt = dict(count=torch.empty(e, dtype=torch.int32, device=dev),
               start=torch.empty(e + 1, dtype=torch.int32, device=dev),
               padded=torch.empty(e, dtype=torch.int32, device=dev),
               sorted_ids=torch.empty(cap, dtype=torch.int32, device=dev),
               dst_row=torch.empty(t * k, dtype=torch.int32, device=dev))
    qa = torch.empty((cap, h), dtype=torch.int8, device=dev)
    ra = torch.empty(cap, dtype=torch.float32, device=dev)
    gu = torch.empty((cap, 2 * inter), dtype=torch.float16, device=dev)
    q2 = torch.empty((cap, inter), dtype=torch.int8, device=dev)
    r2 = torch.empty(cap, dtype=torch.float32, device=dev)
    y = torch.empty((cap, h), dtype=torch.float16, device=dev)
    out = torch.empty((t, h), dtype=torch.float16, device=dev)
    ws = torch.empty(w8a8.moe_gemm_workspace_size(e, cap, h, inter), dtype=torch.uint8, device=dev)
    ws_silu = torch.empty(w8a8.moe_gate_up_silu_workspace_size(cap, inter), dtype=torch.uint8,
                          device=dev)
    sort_ws = torch.empty(max(1, w8a8.moe_sort_workspace_size(t, k, e)), dtype=torch.uint8,
                          device=dev)
    st = {
        "route": lambda: w8a8.topk_softmax(logits, k, out=(rw, rid)),
        "sort": lambda: w8a8.moe_sort(rid, e, 32, workspace=sort_ws, out=srt),
        "quant": lambda: w8a8.moe_smoothquant(x, s, rid, dst_row=srt["dst_row"], rows=cap,
                                              out=qa, row_scale=ra),
        "gate_up_silu": lambda: w8a8.moe_gate_up_silu(qa, wgu_il, srt["start"], srt["count"], ra,
                                                      sgu_il, q=q2, row_scale=r2,
                                                      workspace=ws_silu),
        "gate_up": lambda: w8a8.moe_gemm(qa, wgu, srt["start"], srt["count"], ra, sgu, out=gu,
                                         workspace=ws),
        "silu_quant": lambda: w8a8.moe_silu_mul_quant(gu, srt["start"], srt["count"], q=q2,
                                                      row_scale=r2),
        "down": lambda: w8a8.moe_gemm(q2, wd, srt["start"], srt["count"], r2, sd, out=y,
                                      workspace=ws),
        "combine": lambda: w8a8.moe_combine(y, rw, srt["dst_row"], out=out),
    }
    stages = ["route", "sort", "quant", "gate_up_silu", "down", "combine"]
    stages_u = ["route", "sort", "quant", "gate_up", "silu_quant", "down", "combine"]
    fused = [st[n] for n in stages]
    unfused = [st[n] for n in stages_u]

    for c in fused:  # eager reference layer
        c()
    torch.cuda.synchronize()
    ref = out.clone()
    t_end = time.perf_counter() + 0.3
    while time.perf_counter() < t_end:
        for c in fused + unfused:
            c()
        torch.cuda.synchronize()
    gf, sf = capture_graph(torch, fused, iters)
    gu_, su = capture_graph(torch, unfused, iters)
    tf, tu = [], []
    for rnd in range(rounds):
        for g, stm, dst in ((gf, sf, tf), (gu_, su, tu))[::(1 if rnd % 2 == 0 else -1)]:
            dst.append(replay_us(torch, g, stm) / iters)
    gf.replay()  # the last replay: the fused layer's output
    torch.cuda.synchronize()
    same = bool(torch.equal(out.view(torch.int16), ref.view(torch.int16)))
    per = {}
    for n in dict.fromkeys(stages + stages_u):
        g, stm = capture_graph(torch, [st[n]], iters)
        per[n] = min(replay_us(torch, g, stm) for _ in range(3)) / iters
        del g
    total_us = sum(tf) / len(tf)
    unf_total = sum(tu) / len(tu)
    rows = t * k
    ops_gu = 2.0 * rows * 2 * inter * h
    ops_d = 2.0 * rows * h * inter
    return {"workload": "cfg5 MoE FFN, Mixtral-8x7B shape: 4096 tokens, hidden 4096, ffn 14336, "
                        "8 experts, top-2 (routing -> sort -> quant -> gate_up GEMM with the "
                        "SiLU*up epilogue + requant -> down -> combine)",
            "timing": f"graph replays of {iters} layers, {rounds} replays per form alternating; "
                      f"stages each in a graph of {iters} launches (best of 3 replays)",
            "us_per_layer": total_us, "us_per_layer_replays": tf,
            "TOPS": (ops_gu + ops_d) / (total_us * 1e-6) / 1e12,
            "graph_matches_eager": same,
            "stage_us": {n: per[n] for n in stages},
            "unfused_us_per_layer": unf_total,
            "unfused_stage_us": {n: per[n] for n in stages_u},
            "fused_saving_us": unf_total - total_us,
            "gate_up_silu_TOPS": ops_gu / (per["gate_up_silu"] * 1e-6) / 1e12,
            "down_TOPS": ops_d / (per["down"] * 1e-6) / 1e12,
            "frac_mfma": (ops_gu + ops_d) / (total_us * 1e-6) / PEAK_INT8_OPS,
            "cpu_baseline": (cpu_baseline_moe(*(v.cpu().numpy() for v in
                                                (x, logits, s, wgu, sgu, wd, sd)), k)
                             if cpu else None)}


def bench_hipblaslt_yardstick(torch, projs, iters=10):
    """Same-box yardstick: hipBLASLt's int8 GEMM (torch._int_mm, int32 output,
    no quantizer and no dequant) on the cfg3 projections, in TOPS."""
    out = []
    for (name, k, n), p in zip(LLAMA3_8B, projs):
        a, bt = p["q"], p["w"].t()  # [M, K] and the [K, N] view of the [N, K] weights
        for _ in range(3):
            torch._int_mm(a, bt)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            torch._int_mm(a, bt)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / iters
        out.append({"proj": name, "K": k, "N": n, "us": us,
                    "TOPS": 2.0 * p["m"] * n * k / (us * 1e-6) / 1e12})
    return out


def board_power(torch, dev, loads, secs=2.0, lead=1.0, every=0.02):
    """Socket power and GFX clock read through amdsmi (read-only queries; no
    setting is changed) every `every` s while each callable of `loads` runs
    back to back for `lead` + `secs` s, sampled over the last `secs` (the
    reported power follows a load change with a lag of about a second):
    medians and 90th percentiles per load, with the board's power cap.  The GPU is matched to the amdsmi handle by PCI bus id.
    Empty when amdsmi is not importable or reports no matching GPU."""
    try:
        import amdsmi
    except ImportError:
        return {"note": "amdsmi not importable"}
    import statistics
    import threading

    try:
        amdsmi.amdsmi_init()
    except Exception as e:  # no driver interface visible: nothing to report
        return {"note": f"amdsmi_init failed: {e}"[:200]}
    try:
        props = torch.cuda.get_device_properties(dev)
        want = getattr(props, "pci_bus_id", None)
        handle = None
        for h in amdsmi.amdsmi_get_processor_handles():
            bdf = amdsmi.amdsmi_get_gpu_device_bdf(h)  # dddd:bb:dd.f
            if want is None or int(bdf.split(":")[1], 16) == want:
                handle = h
                break
        if handle is None:
            return {"note": "no amdsmi handle with this GPU's PCI bus id"}
        cap = amdsmi.amdsmi_get_power_cap_info(handle).get("power_cap")
        out = {"power_cap_W": cap / 1e6 if isinstance(cap, (int, float)) else None,
               "note": f"amdsmi current_socket_power and GFX clock sampled every {every * 1e3:.0f} ms "
                       f"over {secs:.1f} s, after each load had run {lead:.1f} s"}
        for name, fn in loads.items():
            watts, mhz, stop = [], [], [False]

            def sample():
                while not stop[0]:
                    try:
                        w = amdsmi.amdsmi_get_power_info(handle).get("current_socket_power")
                        c = amdsmi.amdsmi_get_clock_info(handle, amdsmi.AmdSmiClkType.GFX).get("clk")
                        if isinstance(w, (int, float)):
                            watts.append(w)
                        if isinstance(c, (int, float)):
                            mhz.append(c)
                    except Exception:  # a failed query drops one sample
                        pass
                    time.sleep(every)

            t_lead = time.perf_counter() + lead
            while time.perf_counter() < t_lead:
                fn()
            th = threading.Thread(target=sample, daemon=True)
            th.start()
            t_end = time.perf_counter() + secs
            while time.perf_counter() < t_end:
                fn()
            torch.cuda.synchronize()
            stop[0] = True
            th.join()
            q90 = lambda v: sorted(v)[int(0.9 * (len(v) - 1))] if v else None
            out[name] = {"socket_W_median": statistics.median(watts) if watts else None,
                         "socket_W_p90": q90(watts),
                         "gfx_MHz_median": statistics.median(mhz) if mhz else None,
                         "samples": len(watts)}
        return out
    finally:
        amdsmi.amdsmi_shut_down()


def measured_peaks(torch, dev, cus):
    """Ceilings measured on this GPU in this run (libw8a8_peaks.so, built from
    csrc/peaks.hip): the int8 MFMA-only loop (random and zero operands), the
    LDS read rate per CU, a streaming copy over 2 x 1 GiB, and the launch floor of back-to-back
    launches replayed from a graph (48 per replay, as the cfg1 quantizer is
    timed)."""
    import ctypes

    lib_path = ROOT / "optimized_rocwmma_samples_amd" / "lib" / "libw8a8_peaks.so"
    lib = ctypes.CDLL(str(lib_path))
    lib.w8a8_peak_mfma_ops.restype = ctypes.c_double
    lib.w8a8_peak_mfma_ops.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
    lib.w8a8_peak_mfma.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p,
                                   ctypes.c_void_p]
    lib.w8a8_peak_stream.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
                                     ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_void_p, ctypes.c_void_p]
    lib.w8a8_peak_empty.argtypes = [ctypes.c_void_p]

    def check(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: hipError {rc}")

    def timed(launch, reps):
        st = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(2):
            launch(st.cuda_stream)
        e0.record(st)
        for _ in range(reps):
            launch(st.cuda_stream)
        e1.record(st)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / reps  # seconds per launch

    out = {}
    blocks, iters = cus, 4096
    sink = torch.empty(blocks * 8, dtype=torch.int32, device=dev)
    ops = lib.w8a8_peak_mfma_ops(blocks, iters)
    # mode bit 0: random operands, bit 1: the 16x16x64 form (the GEMM's)
    for key, mode in (("mfma_i8_random_TOPS", 1), ("mfma_i8_zeros_TOPS", 0),
                      ("mfma16_i8_random_TOPS", 3), ("mfma16_i8_zeros_TOPS", 2)):
        t_end = time.perf_counter() + 0.2  # let the clocks settle under this load
        while time.perf_counter() < t_end:
            check(lib.w8a8_peak_mfma(blocks, iters, mode, sink.data_ptr(),
                                     torch.cuda.current_stream(dev).cuda_stream), "peak_mfma")
            torch.cuda.synchronize()
        sec = timed(lambda s, md=mode: check(lib.w8a8_peak_mfma(blocks, iters, md, sink.data_ptr(),
                                                                s), "peak_mfma"), 10)
        out[key] = ops / sec / 1e12
    out["mfma_note"] = (f"MFMA-only loops of the same ops, {blocks} blocks: 4 waves x 8 "
                        f"accumulators x {iters} rounds of v_mfma_i32_32x32x32_i8, or 8 waves "
                        f"(the GEMM's two per SIMD) x 16 accumulators x {iters // 2} rounds of "
                        "v_mfma_i32_16x16x64_i8; operands held in registers")
    # LDS read ceiling: ds_read_b128 only, conflict-free, one block per CU;
    # bytes per shader clock per CU from each CU's slowest wave (s_memtime)
    lib.w8a8_peak_lds.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lds_iters = 4096
    cyc = torch.zeros(cus * 16, dtype=torch.int64, device=dev)
    lsink = torch.empty(cus * 1024, dtype=torch.int32, device=dev)
    lds = {}
    for th in (256, 512, 1024):
        waves = th // 64
        sec = timed(lambda s, th=th: check(lib.w8a8_peak_lds(cus, th, lds_iters, cyc.data_ptr(),
                                                             lsink.data_ptr(), s), "peak_lds"), 5)
        slowest = cyc.view(cus, 16)[:, :waves].max(dim=1).values.double()
        lds[f"{waves}_waves"] = {
            "B_per_clk_per_CU": float((waves * lds_iters * 1024 / slowest).median()),
            "chip_TBps": cus * waves * lds_iters * 1024 / sec / 1e12}
    out["lds_read"] = lds
    out["lds_read_note"] = ("ds_read_b128 loop (64 lanes on 64 consecutive 16-byte chunks, no "
                            "bank conflicts), one block of 4/8/16 waves per CU, 4096 reads per "
                            "lane; bytes per shader clock per CU from s_memtime over each CU's "
                            "slowest wave (median over CUs), chip rate from events")
    del cyc, lsink
    nbytes = 1 << 30
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(3)
    dst = torch.empty_like(src)

    def stream(s, src_p, dst_p, size, b, th, var, md):
        check(lib.w8a8_peak_stream(src_p, dst_p, size, b, th, var, md, sink.data_ptr(), s),
              "peak_stream")

    # best over the stream forms (grid-stride or contiguous per block, 8 or 16
    # loads in flight per lane, plain or non-temporal loads) and launch shapes
    shapes = [(cus * bpc, th) for bpc in (1, 2, 4, 8) for th in (256, 512, 1024)
              if bpc * th <= 2048]
    for mode, key, moved in ((0, "read_GBps", 1.0), (1, "copy_GBps", 2.0),
                             (2, "stream21_GBps", 1.5)):
        best, arg = 0.0, None
        for var in range(8):
            for b, th in shapes:
                sec = timed(lambda s, b=b, th=th, v=var, md=mode: stream(
                    s, src.data_ptr(), dst.data_ptr(), nbytes, b, th, v, md), 6)
                rate = moved * nbytes / sec / 1e9
                if rate > best:
                    best, arg = rate, (var, b, th)
        out[key] = best
        out[key.replace("_GBps", "_form")] = {"variant": arg[0], "blocks": arg[1],
                                              "threads": arg[2]}
    out["stream_note"] = ("2^30 bytes read per launch; copy writes 2^30, stream21 writes 2^29 "
                          "(the quantizer's 2:1 ratio); 16 B per lane access; best over 8 forms "
                          "(variant bits: 0 contiguous range per block, 1 sixteen loads in "
                          "flight per lane instead of eight, 2 non-temporal loads) and "
                          f"{len(shapes)} launch shapes of 1-8 blocks per CU x 256-1024 threads")
    # an independent yardstick: torch's own device-to-device copy
    sec = timed(lambda s: dst.copy_(src), 6)
    out["torch_copy_GBps"] = 2.0 * nbytes / sec / 1e9
    out["torch_copy_note"] = "dst.copy_(src) over 2^30 bytes (read + write counted)"
    del src, dst
    # the 2:1 stream at the cfg1 quantizer's size and launch pattern: 24 buffer
    # pairs (MALL-cold) used in turn, 48 launches replayed from a graph; best
    # over the forms and shapes that suit a 16.8 MB launch
    m1, n1 = 2048, 4096
    pairs = [(torch.empty(2 * m1 * n1, dtype=torch.uint8, device=dev).fill_(1),
              torch.empty(m1 * n1, dtype=torch.uint8, device=dev)) for _ in range(24)]
    best, arg = 0.0, None
    for var in (0, 1, 3, 5, 7):
        for b, th in ((cus, 256), (cus, 512), (cus, 1024), (cus * 2, 256), (cus * 2, 512),
                      (cus * 4, 256)):
            calls = [(lambda p=pairs[i % 24], b=b, th=th, v=var: stream(
                torch.cuda.current_stream(dev).cuda_stream, p[0].data_ptr(), p[1].data_ptr(),
                2 * m1 * n1, b, th, v, 2)) for i in range(48)]
            rate = 3 * m1 * n1 / (graph_us(torch, calls) * 1e-6) / 1e9
            if rate > best:
                best, arg = rate, (var, b, th)
    out["stream21_cfg1_GBps"] = best
    out["stream21_cfg1_form"] = {"variant": arg[0], "blocks": arg[1], "threads": arg[2]}
    out["stream21_cfg1_note"] = ("2:1 stream of cfg1's bytes (16.8 MB read, 8.4 MB written), "
                                 "24 buffer pairs in turn, 48 graph-replayed launches: the "
                                 "quantizer's cold cfg1 measurement with the arithmetic removed; "
                                 "best of 5 forms x 6 launch shapes")
    del pairs
    # a read-only stream of one cfg4 weight matrix (28672 x 8192 bytes), two
    # copies alternating (MALL-cold) in 20 graph-replayed launches: the decode
    # GEMM's measurement with everything but the weight stream removed
    wb = 28672 * 8192
    bufs = [torch.empty(wb, dtype=torch.uint8, device=dev).fill_(2) for _ in range(2)]
    best, arg = 0.0, None
    for var in (1, 3, 5, 7):
        for b, th in ((cus, 256), (cus, 512), (cus * 2, 256), (cus * 4, 256)):
            calls = [(lambda bb=bufs[i % 2], b=b, th=th, v=var: stream(
                torch.cuda.current_stream(dev).cuda_stream, bb.data_ptr(), bb.data_ptr(), wb, b,
                th, v, 0)) for i in range(20)]
            rate = wb / (graph_us(torch, calls) * 1e-6) / 1e9
            if rate > best:
                best, arg = rate, (var, b, th)
    out["read_cfg4_GBps"] = best
    out["read_cfg4_form"] = {"variant": arg[0], "blocks": arg[1], "threads": arg[2]}
    out["read_cfg4_note"] = ("read-only stream of 235 MB (one cfg4 weight matrix), two copies in "
                             "turn, 20 graph-replayed launches: the decode layers' measurement "
                             "with the activations, MFMAs and outputs removed; best of 4 forms x "
                             "4 launch shapes")
    del bufs
    calls = [lambda: check(lib.w8a8_peak_empty(torch.cuda.current_stream(dev).cuda_stream),
                           "peak_empty")] * 48
    out["launch_floor_us"] = graph_us(torch, calls)
    out["launch_floor_note"] = "empty kernel, 48 launches per captured-graph replay"
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="untimed steps for at least this long before the warmup steps "
                         "(the GPU's clocks ramp up from idle)")
    ap.add_argument("--m", type=int, default=8192, help="tokens per projection")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=256)
    ap.add_argument("--no-extras", action="store_true", help="skip cfg1/cfg2 side measurements")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 1 GiB device copy (reads 1 GiB, writes 1 GiB) so "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE can be scaled to bytes")
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the W8A8 path is a "
                          "single-GPU kernel path (run with --gpus 1)", "n_gpus": args.gpus}))
        return 2

    import torch

    import optimized_rocwmma_samples_amd as w8a8

    w8a8.library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x5EED0003)

    log(f"{w8a8.version()} on {torch.cuda.get_device_name(dev)}")
    projs = [make_projection(torch, dev, args.m, k, n) for (_, k, n) in LLAMA3_8B]
    log("cfg3 inputs generated (datagen streams, seed 0x5EED0003)")
    total_ops = sum(2.0 * p["m"] * p["n"] * p["k"] for p in projs)

    def step(events=None):
        for i, p in enumerate(projs):
            if events is not None:
                events[i][0].record()
            w8a8.smoothquant(p["x"], p["s"], out=p["q"], row_scale=p["r"])
            if events is not None:
                events[i][1].record()
            w8a8.gemm(p["q"], p["w"], p["r"], p["sb"], out=p["c"])
            if events is not None:
                events[i][2].record()

    # The GPU raises its clocks from idle over some tens of ms: a cold start's
    # first 10 steps take ~2.1 ms each against ~1.58 ms once settled (50 ms
    # in).  The step runs untimed for at least --settle-ms before the W
    # warmup steps, so the timed steps see the steady state a continuously
    # loaded GPU runs at.
    t_settle = time.perf_counter() + args.settle_ms / 1e3
    settle_steps = 0
    while time.perf_counter() < t_settle:
        step()
        torch.cuda.synchronize()
        settle_steps += 1
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"settle ({settle_steps} steps, {args.settle_ms:.0f} ms) and warmup done")

    # timed region: exactly `steps` steps, synchronized on both sides
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(args.steps):
        step()
    t1.record()
    torch.cuda.synchronize()
    ms_per_step = t0.elapsed_time(t1) / args.steps
    value = total_ops / (ms_per_step * 1e-3) / 1e12
    log(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step, {value:.1f} TOPS")

    # per-kernel durations (separate pass with an event around every launch)
    ev = [[[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in projs]
          for _ in range(args.steps)]
    for s in range(args.steps):
        step(ev[s])
    torch.cuda.synchronize()
    q_ms = [0.0] * len(projs)
    g_ms = [0.0] * len(projs)
    for s in range(args.steps):
        for i in range(len(projs)):
            q_ms[i] += ev[s][i][0].elapsed_time(ev[s][i][1]) / args.steps
            g_ms[i] += ev[s][i][1].elapsed_time(ev[s][i][2]) / args.steps
    gemm_ops = [2.0 * p["m"] * p["n"] * p["k"] for p in projs]
    gemm_avg_us = sum(g_ms) / len(g_ms) * 1e3
    gemm_tops = sum(gemm_ops) / (sum(g_ms) * 1e-3) / 1e12
    per_proj = []
    for (name, k, n), p, qm, gm, ops in zip(LLAMA3_8B, projs, q_ms, g_ms, gemm_ops):
        qbytes = 3 * p["m"] * k + 4 * k + 4 * p["m"]
        per_proj.append({"proj": name, "K": k, "N": n, "quant_us": qm * 1e3,
                         "quant_GBps": qbytes / (qm * 1e-3) / 1e9, "gemm_us": gm * 1e3,
                         "gemm_TOPS": ops / (gm * 1e-3) / 1e12})
    log(json.dumps(per_proj))

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    traffic, traffic_per, traffic_by_order = profiled_traffic(projs, cus)
    kinds = [projection_kernel(p, cus) for p in projs]
    algo_bytes = [p["m"] * p["k"] + p["n"] * p["k"] + 2 * p["m"] * p["n"] + 4 * (p["m"] + p["n"])
                  for p in projs]
    roofline = {"bound": "mfma", "achieved": gemm_tops, "peak": PEAK_INT8_OPS / 1e12,
                "unit": "TOPS", "frac": gemm_tops * 1e12 / PEAK_INT8_OPS, "traffic": traffic,
                "traffic_per_projection": traffic_per,
                "algorithmic_bytes_per_projection": algo_bytes,
                "traffic_source": (f"{TRAFFIC_PROFILE.relative_to(ROOT)} (rocprofv3 FETCH_SIZE x2.0 "
                                   "+ WRITE_SIZE x1.0, calibrated on a 2^30-byte copy; "
                                   "FETCH_SIZE includes MALL hits)") if traffic else None,
                "kernel": " + ".join(
                    f"{'gemm_i8_persist_kernel<Cfg<256,256,128,2,2,4,4,16>>' if kd == 'persist' else 'gemm_i8_tile_kernel<Cfg<256,256,128,2,2,4,4,16>, F16>'} ({', '.join(nm for (nm, _, _), k2 in zip(LLAMA3_8B, kinds) if k2 == kd)})"
                    for kd in dict.fromkeys(kinds)),
                "traffic_note": ("per-projection entries of the persistent kernel from its "
                                 "dispatches by position in each step's launch order (qkv, "
                                 "o_proj, gate_up)" if traffic_by_order else
                                 "per-projection entries of the persistent kernel are its average "
                                 "over the projections it runs (one block per CU each)"),
                "avg_launch_us": gemm_avg_us,
                "avg_launch_us_per_kernel": {
                    kd: sum(g for g, k2 in zip(g_ms, kinds) if k2 == kd) * 1e3
                        / sum(1 for k2 in kinds if k2 == kd)
                    for kd in dict.fromkeys(kinds)},
                "note": "int8 ops (2*M*N*K) per launch / average launch duration over the four "
                        "projection GEMMs; peak = 5.0 POP/s dense int8"}

    peaks = measured_peaks(torch, dev, cus)
    log(json.dumps(peaks))
    for pp in per_proj:
        pp["quant_frac_stream21_measured"] = pp["quant_GBps"] / peaks["stream21_GBps"]
    roofline["peak_measured"] = peaks["mfma16_i8_random_TOPS"]
    roofline["frac_measured"] = gemm_tops / peaks["mfma16_i8_random_TOPS"]
    roofline["peak_measured_note"] = ("MFMA-only loop of the GEMM's instruction "
                                      "(v_mfma_i32_16x16x64_i8) on random operands, same run "
                                      "(measured_peaks); the 32x32x32 form's loop: "
                                      "frac_measured_mfma32")
    roofline["frac_measured_mfma32"] = gemm_tops / peaks["mfma_i8_random_TOPS"]

    extras = {}
    if not args.no_extras:
        # the step and the MFMA-only loop of the GEMM's instruction (random
        # operands) against the board's power cap
        import ctypes

        plib = ctypes.CDLL(str(ROOT / "optimized_rocwmma_samples_amd" / "lib" / "libw8a8_peaks.so"))
        plib.w8a8_peak_mfma.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int,
                                        ctypes.c_void_p, ctypes.c_void_p]
        psink = torch.empty(cus * 8, dtype=torch.int32, device=dev)

        def mfma_loop():
            st = torch.cuda.current_stream(dev).cuda_stream
            for _ in range(8):
                if plib.w8a8_peak_mfma(cus, 4096, 3, psink.data_ptr(), st) != 0:
                    raise RuntimeError("w8a8_peak_mfma failed")
            torch.cuda.synchronize()

        def step_sync():
            step()
            torch.cuda.synchronize()

        extras["board_power"] = board_power(torch, dev, {"cfg3_step": step_sync,
                                                         "mfma16_random_loop": mfma_loop})
        log(json.dumps(extras["board_power"]))
        cpu_x = not args.no_cpu_baseline
        extras["smoothquant_cfg1"] = bench_quantizer(torch, w8a8, dev, gen, cpu=cpu_x)
        q1 = extras["smoothquant_cfg1"]
        q1["frac_stream21_cfg1_measured"] = q1["GBps"] / peaks["stream21_cfg1_GBps"]
        q1["frac_stream21_measured"] = q1["GBps"] / peaks["stream21_GBps"]
        log(json.dumps(extras["smoothquant_cfg1"]))
        extras["smoothquant_sweep"] = bench_quantizer_sweep(torch, w8a8, dev, gen)
        log(json.dumps(extras["smoothquant_sweep"]))
        extras["rmsnorm_smoothquant"] = bench_rmsnorm_sq(torch, w8a8, dev, gen)
        log(json.dumps(extras["rmsnorm_smoothquant"]))
        extras["hipblaslt_int_mm_cfg3"] = bench_hipblaslt_yardstick(torch, projs)
        log(json.dumps(extras["hipblaslt_int_mm_cfg3"]))
        extras["gemm_cfg2"] = bench_gemm_4096(torch, w8a8, dev, gen)
        log(json.dumps(extras["gemm_cfg2"]))
        extras["cfg3_smaller_m"] = bench_cfg3_smaller_m(torch, w8a8, dev, projs)
        log(json.dumps(extras["cfg3_smaller_m"]))
        extras["decode_cfg4"] = bench_decode(torch, w8a8, dev, gen, cpu=cpu_x)
        for layer in extras["decode_cfg4"]["layers"]:
            layer["frac_read_cfg4_measured"] = layer["GBps"] / peaks["read_cfg4_GBps"]
        log(json.dumps(extras["decode_cfg4"]))
        extras["moe_cfg5"] = bench_moe(torch, w8a8, dev, gen, cpu=cpu_x)
        log(json.dumps(extras["moe_cfg5"]))

    if args.calibrate_copy:
        src = torch.randint(-127, 128, (1 << 30,), generator=gen, device=dev, dtype=torch.int8)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)  # elementwise kernel: 2^30 bytes in, 2^30 bytes out
        torch.cuda.synchronize()
        log("calibration copy: 1073741824 bytes read + 1073741824 bytes written (torch neg)")
        del src, dst

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(projs, args.cpu_rows)
        log(json.dumps(cpu))

    line = {
        "metric": "int8 TOPS (%MFMA peak) fused SQ+GEMM; SmoothQuant GB/s (%HBM peak)",
        "value": value,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": args.settle_ms,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: the seeded counter-based streams of datagen.py (N(0,1) "
                "activations with 0.5% x20 outlier columns, U[0.5,2] smooth scale, "
                "U{-127..127} int8 weights, U[1e-3,1e-2] channel scales), the cfg3 parity "
                "tests' inputs",
        "config": {"workload": "cfg3 fused SmoothQuant + W8A8 GEMM, Llama-3-8B projections "
                               "qkv/o_proj/gate_up/down",
                   "m": args.m, "projections": [[n_, k, n] for (n_, k, n) in LLAMA3_8B],
                   "parallelism": "single GPU"},
        "frac_mfma_peak": value * 1e12 / PEAK_INT8_OPS,
        "roofline": roofline,
        "measured_peaks": peaks,
        "cpu_baseline": cpu,
        "per_projection": per_proj,
        **extras,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
