"""Profiling driver: a few FT steps of one workload plus a calibration copy.

Meant to run under `rocprofv3 --pmc ...` (or --kernel-trace).  After the FT
steps it copies a 1 GiB float32 buffer once with torch (`dst.copy_(src)`), a
kernel whose true HBM traffic is known (1 GiB read + 1 GiB written), so the
FETCH_SIZE / WRITE_SIZE a counter pass reports for the FT kernels can be
scaled by what the same counters read for that copy.

  python stockfish-trainer_amd/sft_amd/profile_step.py --workload 1 --steps 3 [--bwd atomic]
"""

from __future__ import annotations

import argparse
import os
import sys

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

import torch  # noqa: E402

from sft_amd import _native, workloads  # noqa: E402
from sft_amd.quantized import QuantizedFeatureTransformer  # noqa: E402
from src.model.modules.feature_transformer import SparseLinearFunction  # noqa: E402
from src.model.modules.feature_transformer import kernel as ftk  # noqa: E402

CALIB_BYTES = 1 << 30


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--bwd", choices=["sorted", "atomic"], default="sorted")
    args = ap.parse_args()
    dev = torch.device("cuda:0")
    _native.lib()
    w = workloads.WORKLOADS[args.workload]
    print(f"[profile] {w.name} B={w.B} N={w.N} K={w.K} L={w.L}", flush=True)
    if w.quantized:
        d = workloads.make_q16_inputs(w)
        d["idx_b"] = workloads.make_indices(workloads.rng(w.wid, workloads.S_BLACK), w.B, w.N, w.K, w.lo, w.hi)
        iw = torch.from_numpy(d["idx_w"]).to(dev)
        ib = torch.from_numpy(d["idx_b"]).to(dev)
        qft = QuantizedFeatureTransformer(*(torch.from_numpy(d[k]).to(dev) for k in ("Wq", "bq", "psqt")), 0, 127)
        for _ in range(args.steps + 1):
            qft(iw, ib)
    else:
        d = workloads.make_fp32_inputs(w)
        iw = torch.from_numpy(d["idx_w"]).to(dev)
        ib = torch.from_numpy(d["idx_b"]).to(dev)
        W = torch.from_numpy(d["W"]).to(dev).requires_grad_(True)
        b = torch.from_numpy(d["bias"]).to(dev).requires_grad_(True)
        gw = torch.from_numpy(d["g_w"]).to(dev)
        gb = torch.from_numpy(d["g_b"]).to(dev)
        atomic = args.bwd == "atomic"
        for _ in range(args.steps + 1):
            W.grad = None
            b.grad = None
            ow = SparseLinearFunction.apply(iw, W, b)
            ob = SparseLinearFunction.apply(ib, W, b)
            if atomic:
                k = ftk.make_sparse_input_linear_backward_kernel(w.K, w.L)
                dW = torch.empty_like(W)
                db = torch.empty_like(b)
                k(iw, dW, db, gw, accumulate=False, atomic=True)
                k(ib, dW, db, gb, accumulate=True, atomic=True)
            else:
                torch.autograd.backward([ow, ob], [gw, gb])
    torch.cuda.synchronize()
    src = torch.ones(CALIB_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[profile] done; calibration copy of {CALIB_BYTES} bytes", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
