#!/usr/bin/env python3
"""Record golden vectors from the REFERENCE's own routines (oracle/_ref/libref.so,
compiled from /root/reference by oracle/Makefile) on seeded inputs.

  python tests/golden/make_golden.py --cpu            # gemm_cpu_h fixtures (runs here)
  python tests/golden/make_golden.py --gpu --out DIR  # kernel_smoothquant / kernel_moe_smoothquant /
                                                      # kernel_(add_)rmsnorm2d_fwd outputs
                                                      # recorded on an MI355X
  python tests/golden/make_golden.py --rmsnorm --out DIR  # the RMSNorm ones only

The .npz files hold inputs and expected outputs only (data, no code).  The
CPU oracle tests compare against them (tests/test_oracle_cpu.py).
"""
from __future__ import annotations

import argparse
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import oracle_lib as O  # noqa: E402
from optimized_rocwmma_samples_amd import datagen as G  # noqa: E402


def cpu_fixtures(out: Path) -> None:
    for (m, n, k, layout) in [(13, 11, 48, 0), (32, 24, 160, 0), (9, 17, 64, 1)]:
        seed = 0x60D0 + m * 131 + n * 7 + k + layout
        a = G.int8(seed, G.TID_A, (m, k) if layout == 0 else (k, m))
        b = G.int8(seed, G.TID_B, (n, k) if layout == 0 else (k, n))
        d = O.ref_gemm_cpu_i8(a, b, layout)
        assert d is not None, "oracle/_ref not built (make -C oracle)"
        path = out / f"gemm_cpu_h_{m}x{n}x{k}_l{layout}.npz"
        np.savez_compressed(path, a=a, b=b, d=d, layout=layout)
        print("wrote", path)


def gpu_fixtures(out: Path) -> None:
    import torch

    ref = O.ref()
    assert ref is not None, "oracle/_ref not built"
    dev = torch.device("cuda:0")
    for (m, n) in [(16, 4096), (8, 1000), (4, 8192), (6, 4104)]:
        seed = 0x51A0 + n
        x = G.activations(seed, m, n)
        s = G.uniform(seed, G.TID_S, (n,), 0.5, 2.0)
        xd = torch.from_numpy(x).to(dev)
        sd = torch.from_numpy(s).to(dev)
        q = torch.zeros((m, n), dtype=torch.int8, device=dev)
        r = torch.zeros(m, dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        rc = ref.ref_kernel_smoothquant(xd.data_ptr(), sd.data_ptr(), q.data_ptr(), r.data_ptr(),
                                        m, n, 127.0)
        assert rc == 0, rc
        path = out / f"smoothquant_ref_{m}x{n}.npz"
        np.savez_compressed(path, x=x, s=s, q=q.cpu().numpy(), r=r.cpu().numpy(), m=m, n=n,
                            seed=seed, quant_max=127.0)
        print("wrote", path, flush=True)
    tokens, hidden, experts, topk = 12, 1024, 8, 2
    seed = 0x3E0
    x = G.activations(seed, tokens, hidden)
    s = G.uniform(seed, G.TID_EXPERT_S, (experts, hidden), 0.5, 2.0)
    h = G.hash64(seed, G.TID_LOGITS, 0, tokens * experts).reshape(tokens, experts)
    ids = np.argsort(h, axis=1, kind="stable")[:, :topk].astype(np.int32)
    ids[3, 1] = -1  # invalid id: the reference leaves that row unwritten
    rows = tokens * topk
    xd, sd, idd = (torch.from_numpy(v).to(dev) for v in (x, s, ids))
    q = torch.zeros((rows, hidden), dtype=torch.int8, device=dev)
    r = torch.zeros(rows, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    rc = ref.ref_kernel_moe_smoothquant(xd.data_ptr(), sd.data_ptr(), idd.data_ptr(),
                                        q.data_ptr(), r.data_ptr(), tokens, hidden, topk,
                                        experts, 127.0)
    assert rc == 0, rc
    valid = ((ids >= 0) & (ids < experts)).reshape(-1).astype(np.uint8)
    path = out / f"moe_smoothquant_ref_{tokens}x{hidden}_e{experts}k{topk}.npz"
    np.savez_compressed(path, x=x, s=s, ids=ids, q=q.cpu().numpy(), r=r.cpu().numpy(),
                        valid=valid, quant_max=127.0)
    print("wrote", path, flush=True)


def gpu_rmsnorm_fixtures(out: Path) -> None:
    import torch

    assert O.ref() is not None, "oracle/_ref not built"
    dev = torch.device("cuda:0")
    eps = 1e-5
    # add + rmsnorm: rows of whole 8-element vectors (the reference has no tail)
    for (m, n) in [(8, 4096), (4, 8192), (6, 2048)]:
        seed = 0x4D50 + n
        x, res, gamma = G.rmsnorm_inputs(seed, m, n)
        xo, y = O.ref_rmsnorm2d_gpu(*(torch.from_numpy(v).to(dev) for v in (x, gamma)), eps=eps,
                                    residual=torch.from_numpy(res).to(dev))
        path = out / f"add_rmsnorm2d_ref_{m}x{n}.npz"
        np.savez_compressed(path, x=x, res=res, gamma=gamma, x_out=xo.cpu().numpy(),
                            y=y.cpu().numpy(), eps=eps)
        print("wrote", path, flush=True)
    # plain rmsnorm; N = 1024 is the reference's own sweep size, where its
    # tail loop adds every column twice
    for (m, n) in [(8, 4096), (4, 1024)]:
        seed = 0x4D60 + n
        x, _, gamma = G.rmsnorm_inputs(seed, m, n)
        _, y = O.ref_rmsnorm2d_gpu(*(torch.from_numpy(v).to(dev) for v in (x, gamma)), eps=eps)
        path = out / f"rmsnorm2d_ref_{m}x{n}.npz"
        np.savez_compressed(path, x=x, gamma=gamma, y=y.cpu().numpy(), eps=eps)
        print("wrote", path, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--cpu", action="store_true")
    ap.add_argument("--gpu", action="store_true")
    ap.add_argument("--rmsnorm", action="store_true", help="only the RMSNorm reference fixtures")
    ap.add_argument("--out", default=str(HERE))
    a = ap.parse_args()
    out = Path(a.out)
    out.mkdir(parents=True, exist_ok=True)
    if a.cpu:
        cpu_fixtures(out)
    if a.gpu:
        gpu_fixtures(out)
    if a.gpu or a.rmsnorm:
        gpu_rmsnorm_fixtures(out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
