#!/usr/bin/env python3
"""FT fwd+bwd throughput on one MI355X.

One step = forward and backward of both perspectives through
SparseLinearFunction (two applies sharing W and b, autograd summing the two
dense weight grads), on inputs already resident in HBM, timed as replays of
the step captured in a HIP graph (--no-graph: launched eagerly; the per-kernel
durations always come from an eager pass).  Prints one JSON line:
positions/s of the headline workload (1: B=65536, L=1048), the roofline of its
dominant kernel, a CPU baseline (the PyTorch-CPU restatement timed on a bounded
sample of the same workload) and, under "configs", the same measurements for
every workload 0-4.

Roofline of the dominant kernel (the most time per step among kernels with an
algorithmic byte count): the memory-side bytes the counters report per launch
(rocprofv3 FETCH_SIZE x 2 + WRITE_SIZE, from two passes run in child processes
before this process touches the GPU, or the committed summary) over its average
HIP-event duration, against HBM's published 8 TB/s.  Beside it, as "logical",
the algorithmic bytes of the byte model (every requested row counted, including
the re-reads the L2 serves, so that fraction can exceed 1), and for gathers the
L2-side figures: a derived L2 peak and the measured ceiling of L2-served row
gathers (sft_probe_l2_gather).  Every timed leg is the median of --reps
repetitions of --steps steps, with their minimum and maximum.

  python bench.py [--gpus 1] [--steps 20] [--reps 5] [--warmup 5] [--warmup-s 0.25] [--workload 1]
                  [--bwd sorted|atomic] [--cpu-seconds 12] [--no-cpu] [--no-graph]
                  [--no-configs] [--traffic live|profile|off]
  python bench.py --composed halfka|threats   (module surface, fused vs reference composition)
  python bench.py --transform halfka|threats  (FT + post-FT epilogue, fused vs reference ops)
  python bench.py --optimizer                 (fused Ranger22 update of the FT parameters)
  python bench.py --encode halfka|threats     (GPU feature-index encoder)
  python bench.py --export                    (GPU LEB128 of the .nnue FT weights)
  python bench.py --pipeline                  (host data pipeline + copy + GPU feature encode)
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "stockfish-trainer_amd")
for _p in (PKG, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
METRIC = "FT fwd+bwd positions/sec @B=65536,L1=1040; achieved GB/s vs HBM peak"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def kernel_step_bytes(kind: str, w, idx_pair) -> float | None:
    """Algorithmic bytes one step moves through the kernels of `kind` (both perspectives).

    Gathers: 4 B per index slot, 4*L per gathered or scattered row, 4*L per
    output row (forward) or written weight-grad row (backward); re-layouts:
    the table or grad read once and written once; bias partials: the grad
    read once.  Bytes per launch = this / launches per step.
    """
    from sft_amd import workloads as wl

    if kind in ("fwd_f32_gather", "fwd_f32_tiled_gather"):
        return float(sum(wl.fwd_kernel_bytes(i, w.N, w.L) for i in idx_pair))
    if kind in ("bwd_feature_gather", "bwd_tiled_gather"):
        return float(sum(wl.bwd_gather_kernel_bytes(i, w.N, w.L) for i in idx_pair))
    if kind == "bwd_atomic_scatter":
        return float(sum(wl.fwd_kernel_bytes(i, w.N, w.L) for i in idx_pair))
    if kind == "fwd_tile_relayout":
        return 2 * 2 * 4.0 * w.N * w.L
    if kind == "bwd_bias_partial":
        return 2 * 4.0 * w.B * w.L
    if kind == "fwd_fold_relayout":  # one launch per step: table (+ virtual rows) read, tiles written
        return 4.0 * (2 * w.N + getattr(w, "virtual_rows", 0)) * w.L
    if kind == "bwd_virtual_reduce":  # folded block's grad read, virtual grad written
        return 4.0 * (getattr(w, "folded_rows", 0) + getattr(w, "virtual_rows", 0)) * w.L
    return None


# What the L2 can deliver to the CUs: 8 XCDs x 16 L2 channels x 128 B per clock at
# the 2.4 GHz peak engine clock (the CDNA L2 width; MI355X has 4 MB of L2 per XCD).
# A derived figure, not a published one: reported beside the HBM roofline only.
L2_DERIVED_PEAK_GBS = 8 * 16 * 128 * 2.4

# Kernels that fetch rows at random from a table or grad tile: every byte they
# request passes the L2, whether it hits there or comes from MALL or HBM.
GATHER_KINDS = {"fwd_f32_gather", "fwd_f32_tiled_gather", "bwd_feature_gather", "bwd_tiled_gather",
                "fwd_i16_gather", "fwd_i16_tiled_gather", "bwd_atomic_scatter"}


def roofline(kind: str, bytes_per_launch: float, avg_ms: float, traffic: float | None = None,
             traffic_source: str | None = None, l2_attainable: float | None = None) -> dict:
    """A kernel against HBM's published peak.

    achieved = the memory-side bytes the counters count per launch (`traffic`:
    FETCH_SIZE x 2 + WRITE_SIZE, MALL hits included, so an upper bound of the HBM
    bytes) / the average launch time; frac = achieved / 8 TB/s.  Without counter
    traffic (--traffic off) the algorithmic bytes stand in and the basis says so.
    "logical" prices the algorithmic bytes per launch (the byte model's rows,
    re-reads served by the L2 included) against the same peak; for gathers that
    can exceed 1.  Gathers also get the L2 view: the derived L2 peak and the
    measured ceiling of L2-served 128-byte row gathers."""
    logical = bytes_per_launch / (avg_ms * 1e-3) / 1e9
    r = {"kernel": kind, "bound": "hbm", "peak": HBM_PEAK_GBS, "unit": "GB/s", "avg_launch_ms": avg_ms}
    if traffic:
        hbm = traffic / (avg_ms * 1e-3) / 1e9
        r.update(achieved=hbm, frac=hbm / HBM_PEAK_GBS, traffic=traffic, traffic_source=traffic_source,
                 basis="memory-side bytes per launch (rocprofv3 FETCH_SIZE x 2 + WRITE_SIZE) / average launch time")
    else:
        r.update(achieved=logical, frac=logical / HBM_PEAK_GBS, traffic=None,
                 basis="algorithmic bytes per launch / average launch time (no counter traffic in this run)")
    r["logical"] = {"bytes_per_launch": bytes_per_launch, "achieved": logical,
                    "frac_of_hbm_peak": logical / HBM_PEAK_GBS,
                    "note": "algorithmic bytes of the byte model (4K + 4L(n+1) per position and direction, "
                            "4NL per weight-grad write): every requested row, L2-served re-reads included"}
    if kind in GATHER_KINDS:
        r["l2"] = {"derived_peak": L2_DERIVED_PEAK_GBS, "frac_of_derived_peak": logical / L2_DERIVED_PEAK_GBS,
                   "note": "derived (8 XCDs x 16 channels x 128 B x 2.4 GHz), not a published figure"}
        if l2_attainable:
            r["l2"]["measured_ceiling"] = l2_attainable
            r["l2"]["frac_of_measured_ceiling"] = logical / l2_attainable
    return r


def timed_reps(fn, steps: int, reps: int) -> list:
    """ms per call of fn in each of `reps` repetitions of `steps` back-to-back
    calls, each bracketed by HIP events on the current stream and a
    synchronisation on both sides."""
    import torch

    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    out = []
    for _ in range(reps):
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        out.append(e0.elapsed_time(e1) / steps)
    return out


def rep_stats(ms: list) -> dict:
    """Median (the reported figure), minimum and maximum of the repetitions."""
    import statistics

    return {"ms_per_step": statistics.median(ms), "ms_per_step_min": min(ms), "ms_per_step_max": max(ms),
            "reps": len(ms), "ms_per_step_reps": ms}


def committed_traffic(name: str) -> dict | None:
    """Per-kind memory-side bytes per step of a workload from its committed counter summary."""
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        d = json.load(f)
    d["source"] = os.path.relpath(path, ROOT)
    return d


def live_traffic(wid: int, log_fn) -> dict | None:
    """Both counter passes over the workload, run before this process touches the GPU."""
    import tempfile

    from sft_amd import traffic as tr

    tmp = tempfile.mkdtemp(prefix="sft_pmc_", dir="/tmp")
    try:
        t = tr.measure(wid, tmp, log=log_fn)
    except Exception as e:  # noqa: BLE001 - a failed counter pass leaves traffic unmeasured, not the bench
        log_fn(f"[bench] live counter passes failed: {e}")
        return None
    finally:
        import shutil

        shutil.rmtree(tmp, ignore_errors=True)
    t["source"] = "live: " + "; ".join(t["commands"])
    return t


def l2_gather_ceiling(dev, warmup_s: float) -> dict:
    """Measured ceiling of L2-served 128-byte row gathers: sft_probe_l2_gather over
    a 2 MB table (every XCD's L2 holds it), 8192 workgroups x 32 lane groups x 256
    rows per launch, timed with the library's launch events after a warm-up."""
    import torch

    from sft_amd import _native

    table = torch.randn(1 << 14, 32, device=dev)
    blocks, rounds = 8192, 32
    out = torch.empty(blocks * 1024, device=dev)
    warm_up(lambda: _native.probe_l2_gather(table, rounds, blocks, out), 3, warmup_s)
    _native.prof_enable(True)
    for _ in range(10):
        nbytes = _native.probe_l2_gather(table, rounds, blocks, out)
    torch.cuda.synchronize()
    tot, cnt = _native.prof_collect()["probe_l2_gather"]
    _native.prof_enable(False)
    avg = tot / cnt
    return {"gbs": nbytes / (avg * 1e-3) / 1e9, "kernel": "probe_l2_gather", "table_bytes": table.numel() * 4,
            "bytes_per_launch": nbytes, "avg_launch_ms": avg}


def warm_up(fn, n: int, min_s: float) -> int:
    """Calls fn at least n times and until min_s seconds have passed with the GPU
    busy (a synchronisation every few calls keeps the host clock on the GPU's
    work).  MI355X raises its clocks over the first tens of milliseconds of
    sustained load: a few short warm-up steps leave a short timed region at the
    lower clock (the int16 step: 0.39 ms after 5 warm-up steps, 0.32 ms after
    0.2 s).  Returns the number of calls."""
    import torch

    done = 0
    t0 = time.perf_counter()
    while done < n or time.perf_counter() - t0 < min_s:
        fn()
        done += 1
        if done % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return done


def attainable(dev) -> dict:
    """The measured HBM ceiling beside the 8 TB/s peak: a 1 GiB device-to-device
    copy, bytes read + written per second."""
    import torch

    src = torch.empty(1 << 28, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    return {"copy_gbs": 2 * src.numel() * 4 / (e0.elapsed_time(e1) / 10 * 1e-3) / 1e9, "copy_bytes": 1 << 30}


def cpu_baseline(w, d, seconds: float) -> dict:
    import numpy as np
    import torch

    from oracle.torch_cpu_ft import CpuFtStep

    threads = len(os.sched_getaffinity(0))
    env_threads = os.environ.get("OMP_NUM_THREADS")
    if env_threads and env_threads.isdigit():
        threads = min(threads, int(env_threads))
    torch.set_num_threads(threads)
    Bs = w.B  # the whole batch of the workload, as the GPU step
    step = CpuFtStep(d["idx_w"][:Bs], d["idx_b"][:Bs], d["W"], d["bias"], d["g_w"][:Bs], d["g_b"][:Bs])
    step()  # warm-up
    n, t0 = 0, time.perf_counter()
    while True:
        step()
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 2) or n >= 200:
            break
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    del np
    return {
        "value": Bs * n / el,
        "unit": "positions/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n} fwd+bwd steps of both perspectives on all {Bs} positions of {w.name} "
                  f"(N={w.N}, L={w.L}), torch {torch.__version__} embedding_bag on {threads} threads, "
                  f"{el:.1f} s; cpu: {model}",
    }


def run_q16(args, w, dev, l2_attainable=None, traffic=None) -> dict:
    """int16 inference forward of both perspectives (the quantized workload): one
    step = one tiled int16 gather of both perspectives, PSQT columns included, from
    the table the module packed when it was built (load time, as an engine lays out
    its weights once); the pack's own time is reported beside the step."""
    import torch

    from sft_amd import _native, workloads
    from sft_amd.quantized import QuantizedFeatureTransformer, quantized_ft_forward

    log(f"[bench] generating {w.name}: B={w.B} N={w.N} K={w.K} active U[{w.lo},{w.hi}] L={w.L} int16")
    d = workloads.make_q16_inputs(w)
    d["idx_b"] = workloads.make_indices(workloads.rng(w.wid, workloads.S_BLACK), w.B, w.N, w.K, w.lo, w.hi)
    qft = QuantizedFeatureTransformer(*(torch.from_numpy(d[k]).to(dev) for k in ("Wq", "bq", "psqt")), 0, 127)
    iw = torch.from_numpy(d["idx_w"]).to(dev)
    ib = torch.from_numpy(d["idx_b"]).to(dev)
    warm_up(lambda: qft(iw, ib), args.warmup, args.warmup_s)
    timing = rep_stats(timed_reps(lambda: qft(iw, ib), args.steps, args.reps))
    ms = timing["ms_per_step"]
    _native.prof_enable(True)  # per-kernel durations from a separate pass with the launch events
    for _ in range(args.steps):
        qft(iw, ib)
    torch.cuda.synchronize()
    prof = _native.prof_collect()
    _native.prof_enable(False)
    step_bytes = sum(workloads.q16_fwd_bytes(i, w.N, w.L, w.psqt) for i in (d["idx_w"], d["idx_b"]))
    kern = {k: {"avg_ms": t / c, "launches_per_step": c / args.steps} for k, (t, c) in prof.items()}
    for k, v in kern.items():
        log(f"[bench]   {k:22s} {v['avg_ms']:8.4f} ms x {v['launches_per_step']:.0f}/step")
    gather = [k for k in prof if "i16" in k][0]
    g_avg = prof[gather][0] / prof[gather][1]
    launches = prof[gather][1] / args.steps
    per_launch = step_bytes / launches
    t_launch = None
    if traffic and gather in traffic["kind_step_bytes"]:
        t_launch = traffic["kind_step_bytes"][gather] / launches
    p0 = torch.cuda.Event(enable_timing=True)
    p1 = torch.cuda.Event(enable_timing=True)
    p0.record()
    for _ in range(5):
        qft.repack()
    p1.record()
    torch.cuda.synchronize()
    pack_ms = p0.elapsed_time(p1) / 5

    # The same forward without the kept pack: sft_ft_fwd_i16_ex per perspective,
    # each call re-laying the table out in its workspace.
    def per_call():
        for i in (iw, ib):
            quantized_ft_forward(i, qft.weight_q, qft.bias_q, qft.psqt_q, 0, 127)

    warm_up(per_call, args.warmup, args.warmup_s)
    per_call_ms = rep_stats(timed_reps(per_call, args.steps, args.reps))["ms_per_step"]
    compulsory = workloads.q16_compulsory_bytes(w.B, w.K, w.N, w.L, w.psqt)
    return {
        "workload": w.name, "dtype": "int16", "feature_set": w.feature_set, "batch": w.B, "num_inputs": w.N,
        "max_active": w.K, "active": [w.lo, w.hi], "output_size": w.L, "psqt": w.psqt, "quant_scale": 127,
        "clip": [0, 127], "step": "int16 forward of both perspectives from the packed table",
        **timing, "positions_per_s": w.B / (ms * 1e-3), "step_bytes": step_bytes,
        "step_gbs": step_bytes / (ms * 1e-3) / 1e9,
        "step_compulsory_bytes": compulsory,
        "step_compulsory_frac_of_hbm_peak": compulsory / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "roofline": roofline(gather, per_launch, g_avg, t_launch, traffic["source"] if t_launch else None,
                             l2_attainable),
        "kernels": kern, "pack_ms": pack_ms, "per_call_pack_ms_per_step": per_call_ms,
    }


def bench_q16(args, w, dev) -> int:
    c = run_q16(args, w, dev, traffic=committed_traffic(w.name))
    result = {
        "metric": "int16 FT forward positions/sec (both perspectives) @B=65536,L1=1040",
        "value": c["positions_per_s"], "unit": "positions/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_s": args.warmup_s, "ms_per_step": c["ms_per_step"],
        **{k: c[k] for k in ("reps", "ms_per_step_min", "ms_per_step_max", "ms_per_step_reps")},
        "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int16", "data": "synthetic",
        "config": {"workload": w.name, "feature_set": w.feature_set, "batch": w.B, "num_inputs": w.N,
                   "max_active": w.K, "active": [w.lo, w.hi], "output_size": w.L, "psqt": w.psqt,
                   "quant_scale": 127, "clip": [0, 127], "parallelism": "single-gpu"},
        **{k: c[k] for k in ("step_bytes", "step_gbs", "step_compulsory_bytes", "step_compulsory_frac_of_hbm_peak",
                             "roofline", "kernels", "pack_ms", "per_call_pack_ms_per_step")},
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


COMPOSED = {"halfka": ("HalfKAv2_hm^", 16, 32), "threats": ("Full_Threats+HalfKAv2_hm^", 32, 160)}


def bench_composed(args, dev) -> int:
    """ComposedFeatureTransformer forward + backward of both perspectives at
    B=65536, L=1048 through the module surface: the fused pair op (default)
    timed against the reference composition (merged_weight, then
    SparseLinearFunction per perspective) on the same kernels."""
    import types

    import numpy as np
    import torch

    from sft_amd import _native, workloads
    from src.model.modules.features import get_feature_cls

    name, lo, hi = COMPOSED[args.composed]
    B, L = 65536, 1048
    torch.manual_seed(0)
    ft = get_feature_cls(name)(L).to(dev)
    vrows = folded = 0
    for f in ft.features:
        if hasattr(f, "virtual_weight"):
            with torch.no_grad():
                f.virtual_weight.normal_(0, 0.01)
            vrows += f.virtual_weight.shape[0]
            folded += f.weight.shape[0]
    N, K = ft.NUM_INPUTS, ft.MAX_ACTIVE_FEATURES
    log(f"[bench] composed {name}: B={B} N={N} K={K} active U[{lo},{hi}] L={L}")
    idx = [workloads.make_indices(np.random.default_rng([200 + K, s]), B, N, K, lo, hi) for s in (0, 1)]
    iw, ib = (torch.from_numpy(i).to(dev) for i in idx)
    gw = torch.randn(B, L, device=dev)
    gb = torch.randn(B, L, device=dev)

    def step():
        for p in ft.parameters():
            p.grad = None
        ow, ob = ft(iw, ib)
        torch.autograd.backward([ow, ob], [gw, gb])

    def timed(fused: bool, prof: bool):
        ft.fused = fused
        warm_up(step, args.warmup, args.warmup_s)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        out = None
        if prof:  # per-kernel durations from a separate pass with the launch events
            _native.prof_enable(True)
            for _ in range(args.steps):
                step()
            torch.cuda.synchronize()
            out = _native.prof_collect()
            _native.prof_enable(False)
        return e0.elapsed_time(e1) / args.steps, out

    ref_ms, _ = timed(False, False)
    ms, prof = timed(True, True)
    log(f"[bench] fused {ms:.3f} ms/step, reference composition {ref_ms:.3f} ms/step")
    w = types.SimpleNamespace(N=N, L=L, B=B, virtual_rows=vrows, folded_rows=folded)
    kern = {}
    for kind, (tot, cnt) in prof.items():
        sb = kernel_step_bytes(kind, w, idx)
        per_launch = sb / (cnt / args.steps) if sb else None
        avg = tot / cnt
        kern[kind] = {"avg_ms": avg, "launches_per_step": cnt / args.steps, "bytes_per_launch": per_launch,
                      "gbs": (per_launch / (avg * 1e-3) / 1e9) if per_launch else None}
        log(f"[bench]   {kind:22s} {avg:8.4f} ms x {cnt / args.steps:.0f}/step")
    # dominant kernel: the largest time per step among those with an algorithmic byte count
    dom = max((k for k in prof if kern[k]["bytes_per_launch"]), key=lambda k: prof[k][0])
    dom_avg = prof[dom][0] / prof[dom][1]
    dom_bytes = kern[dom]["bytes_per_launch"]
    step_bytes = workloads.step_bytes(idx[0], idx[1], N, L)
    result = {
        "metric": "composed FT module fwd+bwd positions/sec @B=65536,L1=1040",
        "value": B / (ms * 1e-3), "unit": "positions/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_s": args.warmup_s, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": f"composed_{args.composed}_b65536", "feature_set": name, "batch": B,
                   "num_inputs": N, "virtual_rows": vrows, "max_active": K, "active": [lo, hi],
                   "output_size": L, "parallelism": "single-gpu"},
        "reference_composition": {"ms_per_step": ref_ms, "value": B / (ref_ms * 1e-3)},
        "speedup_vs_reference_composition": ref_ms / ms,
        "step_bytes": step_bytes,
        "step_gbs": step_bytes / (ms * 1e-3) / 1e9,
        "roofline": roofline(dom, dom_bytes, dom_avg),
        "kernels": kern,
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def bench_transform(args, dev) -> int:
    """NNUEModel._transform_inputs forward + backward (FT of both perspectives
    and the post-FT epilogue) at B=65536, L1=1040, 8 PSQT buckets, three ways on
    the same kernels: the reference ops over the reference composition, the
    reference ops over the fused composed op, and the fused transform."""
    import types

    import numpy as np
    import torch

    from sft_amd import _native, workloads
    from src.model.modules.features import get_feature_cls
    from src.model.transform_inputs import transform_inputs

    name, lo, hi = COMPOSED[args.transform]
    B, L1, P = 65536, 1040, 8
    L = L1 + P
    torch.manual_seed(0)
    ft = get_feature_cls(name)(L).to(dev)
    vrows = folded = 0
    with torch.no_grad():
        for f in ft.features:
            f.weight.normal_(0, 0.05)
            if hasattr(f, "virtual_weight"):
                f.virtual_weight.normal_(0, 0.02)
                vrows += f.virtual_weight.shape[0]
                folded += f.weight.shape[0]
        ft.bias.uniform_(0.0, 0.6)
    N, K = ft.NUM_INPUTS, ft.MAX_ACTIVE_FEATURES
    log(f"[bench] transform {name}: B={B} N={N} K={K} active U[{lo},{hi}] L1={L1} P={P}")
    g = np.random.default_rng([300 + K, 0])
    idx = [workloads.make_indices(np.random.default_rng([200 + K, s]), B, N, K, lo, hi) for s in (0, 1)]
    iw, ib = (torch.from_numpy(i).to(dev) for i in idx)
    us = torch.from_numpy(g.integers(0, 2, (B, 1)).astype(np.float32)).to(dev)
    k = torch.from_numpy(g.integers(0, P, B).astype(np.int64)).to(dev)
    g_l0 = torch.randn(B, L1, device=dev)
    g_psqt = torch.randn(B, 1, device=dev)

    def run(mode: str, prof: bool):
        ft.fused = mode != "reference"

        def step():
            for p in ft.parameters():
                p.grad = None
            l0, psqt = transform_inputs(ft, L1, us, iw, ib, k, fused=mode == "fused")
            torch.autograd.backward([l0, psqt], [g_l0, g_psqt])

        warm_up(step, args.warmup, args.warmup_s)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        out = None
        if prof:  # per-kernel durations from a separate pass with the launch events
            _native.prof_enable(True)
            for _ in range(args.steps):
                step()
            torch.cuda.synchronize()
            out = _native.prof_collect()
            _native.prof_enable(False)
        return e0.elapsed_time(e1) / args.steps, out

    ref_ms, _ = run("reference", False)
    f1_ms, _ = run("composed", False)
    ms, prof = run("fused", True)
    log(f"[bench] fused transform {ms:.3f} ms/step; reference ops over the composed op {f1_ms:.3f}; "
        f"over the reference composition {ref_ms:.3f}")
    w = types.SimpleNamespace(N=N, L=L, B=B, virtual_rows=vrows, folded_rows=folded)
    kern = {}
    for kind, (tot, cnt) in prof.items():
        sb = kernel_step_bytes(kind, w, idx)
        if kind == "bwd_epilogue":  # raw tiles and grad tiles of both perspectives + the l0 grad
            sb = 2 * 4.0 * B * L * 2 + 4.0 * B * L1
        per_launch = sb / (cnt / args.steps) if sb else None
        avg = tot / cnt
        kern[kind] = {"avg_ms": avg, "launches_per_step": cnt / args.steps, "bytes_per_launch": per_launch,
                      "gbs": (per_launch / (avg * 1e-3) / 1e9) if per_launch else None}
        log(f"[bench]   {kind:22s} {avg:8.4f} ms x {cnt / args.steps:.0f}/step")
    # dominant kernel: the largest time per step among those with an algorithmic byte count
    dom = max((kk for kk in prof if kern[kk]["bytes_per_launch"]), key=lambda kk: prof[kk][0])
    dom_avg = prof[dom][0] / prof[dom][1]
    dom_bytes = kern[dom]["bytes_per_launch"]
    result = {
        "metric": "FT + post-FT epilogue fwd+bwd positions/sec @B=65536,L1=1040",
        "value": B / (ms * 1e-3), "unit": "positions/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_s": args.warmup_s, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": f"transform_{args.transform}_b65536", "feature_set": name, "batch": B,
                   "num_inputs": N, "virtual_rows": vrows, "max_active": K, "active": [lo, hi], "l1": L1,
                   "psqt_buckets": P, "parallelism": "single-gpu"},
        "reference_ops_over_reference_composition": {"ms_per_step": ref_ms, "value": B / (ref_ms * 1e-3)},
        "reference_ops_over_composed_op": {"ms_per_step": f1_ms, "value": B / (f1_ms * 1e-3)},
        "speedup_vs_reference": ref_ms / ms,
        "roofline": roofline(dom, dom_bytes, dom_avg),
        "kernels": kern,
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def bench_optimizer(args, dev) -> int:
    """Ranger22 full update of the HalfKAv2_hm^ FT parameters (weight
    [24576, 1048], virtual weight [768, 1048], bias [1048]) per step: the fused
    kernel against the reference function's ops run eagerly in torch (the
    reference compiles them with torch.compile, which this build does not use)."""
    import numpy as np
    import torch

    from sft_amd import _native
    from src.ranger22.fused_update import get_fused_full_update

    L = 1048
    shapes = [(24576, L), (768, L), (L,)]
    g = torch.Generator(device=dev).manual_seed(0)
    tensors = []
    for shp in shapes:
        mk = lambda scale: torch.randn(shp, device=dev, generator=g) * scale
        tensors.append([mk(0.05), mk(1e-3), mk(1e-3).abs() * 1e-3, mk(1e-3), mk(1e-3)])
    step, beta1, beta2, lr, eps = 7, 0.9, 0.999, 8.75e-4, 1e-7
    host = [lr, 1 / np.sqrt(1 - beta2 ** step), eps, 2e-4, 1 / np.sqrt((1 + beta2) ** 2 + beta2 ** 2), 2.0, -1.0,
            lr / (1 - beta1 ** step), beta2, 1 - beta2, beta1 * beta1, 1 - beta1 * beta1]
    scalars = torch.tensor(host, dtype=torch.float32, device=dev)

    def reference(p, grad, v, m, mp, s):
        v.mul_(s[8])
        v.add_(grad * grad * s[9])
        m.mul_(s[10])
        m.add_(grad * s[11])
        if p.dim() == 2:
            unorm = torch.linalg.vector_norm(p, ord=2, dim=1, keepdim=True)
        else:
            unorm = torch.linalg.vector_norm(p, ord=2)
        correction = s[3] * (1 - 1 / (unorm + s[2]))
        denom = v.sqrt() * s[1] + s[2]
        pn = (m * s[5] + mp * s[6]) * s[4]
        p.mul_(1 - s[0] * correction)
        p.sub_((pn / denom) * s[7])

    def timed(fn, prof):
        def one():
            for t in tensors:
                fn(*t, scalars)

        warm_up(one, args.warmup, args.warmup_s)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            one()
        e1.record()
        torch.cuda.synchronize()
        out = None
        if prof:  # per-kernel durations from a separate pass with the launch events
            _native.prof_enable(True)
            for _ in range(args.steps):
                one()
            torch.cuda.synchronize()
            out = _native.prof_collect()
            _native.prof_enable(False)
        return e0.elapsed_time(e1) / args.steps, out

    ref_ms, _ = timed(reference, False)
    fused = lambda p, gr, v, m, mp, s: get_fused_full_update(p.dim())(p, gr, v, m, mp, s)
    ms, prof = timed(fused, True)
    elems = sum(int(np.prod(s)) for s in shapes)
    step_bytes = 8 * 4 * elems  # p, grad, v, m, m_prev read; p, v, m written
    tot, cnt = prof["ranger22_update"]
    # the weight table dominates: its launch is the first of each step's three
    big = 8 * 4 * shapes[0][0] * shapes[0][1]
    log(f"[bench] fused Ranger22 update {ms * 1e3:.1f} us/step, reference ops eager {ref_ms * 1e3:.1f} us/step")
    achieved = step_bytes / (tot / cnt * 3 * 1e-3) / 1e9
    result = {
        "metric": "Ranger22 FT-parameter update, GB/s (HalfKAv2_hm^ weight + virtual + bias, L=1048)",
        "value": step_bytes / (ms * 1e-3) / 1e9, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_s": args.warmup_s, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "ranger22_halfka_ft_params", "shapes": shapes, "elements": elems,
                   "parallelism": "single-gpu"},
        "reference_ops_eager": {"ms_per_step": ref_ms, "value": step_bytes / (ref_ms * 1e-3) / 1e9},
        "speedup_vs_reference_ops_eager": ref_ms / ms,
        "roofline": {"kernel": "ranger22_update", "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes_per_step": step_bytes, "weight_table_bytes": big,
                     "avg_launch_ms": tot / cnt},
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def bench_encode(args, dev) -> int:
    """Feature-index encoding of B=65536 positions (both perspectives, index rows
    plus side to move and buckets) on the GPU, positions already in HBM; the C
    oracle on the host cores is the CPU baseline."""
    import os as _os

    import numpy as np
    import torch

    from oracle import feature_oracle
    from sft_amd import _native, positions
    from sft_amd.encode import encode_batch, parse_feature_set

    name = {"halfka": "HalfKAv2_hm", "threats": "Full_Threats+HalfKAv2_hm"}[args.encode]
    B = 65536
    log(f"[bench] encode {name}: generating {B} positions")
    boards_np, stm_np = positions.random_positions(B, seed=7)
    boards = torch.from_numpy(boards_np).to(dev)
    stm = torch.from_numpy(stm_np).to(dev)
    warm_up(lambda: encode_batch(boards, stm, name), args.warmup, args.warmup_s)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        out = encode_batch(boards, stm, name)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    _native.prof_enable(True)  # kernel durations from a separate pass with the launch events
    for _ in range(args.steps):
        out = encode_batch(boards, stm, name)
    torch.cuda.synchronize()
    tot, cnt = _native.prof_collect()["encode_features"]
    _native.prof_enable(False)
    comps, K = parse_feature_set(name)
    active = int((out["white"] >= 0).sum().item() + (out["black"] >= 0).sum().item())
    # algorithmic bytes: boards + side to move read; both index rows, us, psqt and layer-stack buckets written
    step_bytes = B * (64 + 1) + B * (2 * K * 4 + 4 + 8 + 8)
    kern_ms = tot / cnt
    achieved = step_bytes / (kern_ms * 1e-3) / 1e9
    log(f"[bench] encode {ms * 1e3:.1f} us/batch ({B / (ms * 1e-3) / 1e6:.1f} M positions/s), "
        f"{active / B:.1f} features per position")
    cpu = None
    if not args.no_cpu:
        threads = min(len(_os.sched_getaffinity(0)), int(_os.environ.get("OMP_NUM_THREADS", "64")))
        _os.environ["OMP_NUM_THREADS"] = str(threads)
        n = 16384
        comps_names = name.split("+")
        feature_oracle.encode(boards_np[:256], stm_np[:256], comps_names)
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0):
            feature_oracle.encode(boards_np[:n], stm_np[:n], comps_names)
            reps += 1
        el = time.perf_counter() - t0
        cpu = {"value": reps * n / el, "unit": "positions/s", "cores": threads, "kind": "port",
               "sample": f"{reps} x {n} positions of the same batch, oracle/feature_oracle.c with OpenMP, "
                         f"{el:.1f} s"}
        log(f"[bench] cpu baseline {cpu['value'] / 1e6:.2f} M positions/s on {threads} threads")
    result = {
        "metric": f"feature-index encode positions/sec ({name}, both perspectives) @B=65536",
        "value": B / (ms * 1e-3), "unit": "positions/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_s": args.warmup_s, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int32", "data": "synthetic",
        "config": {"workload": f"encode_{args.encode}_b65536", "feature_set": name, "batch": B, "max_active": K,
                   "positions": "random armies (sft_amd.positions.random_positions, seed 7)",
                   "features_per_position": active / B, "parallelism": "single-gpu"},
        "roofline": {"kernel": "encode_features", "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes_per_launch": step_bytes, "avg_launch_ms": kern_ms},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


def bench_export(args, dev) -> int:
    """Signed LEB128 of the exported HalfKAv2_hm FT weights (22528 x 1040 int16,
    the largest tensor of the .nnue file) on the GPU; the per-value loop of the
    reference's encoder (restated in the oracle) on a bounded sample is the CPU
    baseline."""
    import numpy as np
    import torch

    from oracle import leb128_oracle
    from sft_amd import _native

    g = np.random.default_rng(11)
    w = np.clip(np.rint(g.standard_normal((22528, 1040)) * 40), -32768, 32767).astype(np.int16)
    t = torch.from_numpy(w).to(dev)
    warm_up(lambda: _native.leb128_encode(t), args.warmup, args.warmup_s)
    _native.prof_enable(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = _native.leb128_encode(t)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / args.steps
    tot, cnt = _native.prof_collect()["leb128_encode"]
    _native.prof_enable(False)
    kern = tot / cnt
    n = w.size
    nbytes = int(out.numel())
    algo = n * 2 + nbytes  # values read, code bytes written
    log(f"[bench] LEB128 {n} int16 -> {nbytes} bytes: kernels {kern * 1e3:.1f} us, call {wall * 1e6:.1f} us")
    cpu = None
    if not args.no_cpu:
        sample = w.reshape(-1)[:200000]
        t0 = time.perf_counter()
        leb128_oracle.encode(sample)
        el = time.perf_counter() - t0
        cpu = {"value": sample.size / el, "unit": "values/s", "cores": 1, "kind": "port",
               "sample": f"{sample.size} values through the per-value loop of the reference encoder (Python), "
                         f"{el:.1f} s"}
    result = {
        "metric": "signed LEB128 encode values/sec (HalfKAv2_hm FT weights 22528 x 1040 int16)",
        "value": n / (kern * 1e-3), "unit": "values/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "warmup_s": args.warmup_s,
        "ms_per_step": kern, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int16",
        "data": "synthetic", "config": {"workload": "leb128_halfka_export_weights", "values": n,
                                        "encoded_bytes": nbytes, "parallelism": "single-gpu"},
        "call_ms_including_length_readback": wall * 1e3,
        "roofline": {"kernel": "leb128_encode", "bound": "hbm", "achieved": algo / (kern * 1e-3) / 1e9,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": algo / (kern * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "traffic": None, "algorithmic_bytes_per_launch": algo, "avg_launch_ms": kern},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    return 0


def bench_pipeline(args, dev) -> int:
    """Host data pipeline -> GPU: entries read from a file of 1 048 576 decoded
    training entries (16 copies of 65 536 random positions), skip filter off,
    per-reader shuffle buffers of 16 384, batches of 65 536 in pinned slabs,
    copied to the GPU and encoded there (Full_Threats+HalfKAv2_hm).  Reports the
    host stream alone and the stream with the copy and the GPU encode."""
    import tempfile

    import numpy as np
    import torch

    from sft_amd import pipeline as pl
    from sft_amd import positions

    B, copies = 65536, 16
    boards, stm = positions.random_positions(B, seed=13)
    e = pl.make_entries(boards, stm, score=np.arange(B) % 2000 - 1000, result=np.arange(B) % 3 - 1, ply=60)
    tmp = tempfile.mkdtemp(prefix="sft_pipe_", dir="/tmp")
    path = os.path.join(tmp, "entries.sftpos")
    pl.write_entries(path, np.concatenate([e] * copies), entries_per_chunk=16384)
    n = B * copies
    try:
        threads = max(1, min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "64"))) - 2)
    except OSError:
        threads = 4

    def run(to_gpu: bool):
        stream = pl.BatchStream([path], B, reader_threads=threads, shuffle_buffer_entries=16384, seed=1,
                                pin_memory=to_gpu, slab_count=4)
        t0 = time.perf_counter()
        got = 0
        for batch in stream:
            if to_gpu:
                batch.to_device(dev, "Full_Threats+HalfKAv2_hm")
            got += batch.size
            batch.release()
        if to_gpu:
            torch.cuda.synchronize()
        el = time.perf_counter() - t0
        stream.close()
        assert got == n
        return n / el

    host_rate = run(False)
    run(True)  # warm-up of the encode path
    gpu_rate = run(True)
    import shutil

    shutil.rmtree(tmp, ignore_errors=True)
    log(f"[bench] pipeline: host stream {host_rate / 1e6:.2f} M entries/s, with GPU encode {gpu_rate / 1e6:.2f} M/s "
        f"({threads} reader threads)")
    result = {
        "metric": "training entries/sec through the host pipeline + GPU feature encode (Full_Threats+HalfKAv2_hm)",
        "value": gpu_rate, "unit": "entries/s", "n_gpus": 1, "steps": 1, "warmup": 1, "ms_per_step": B / gpu_rate * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int32", "data": "synthetic",
        "config": {"workload": "pipeline_threats_b65536", "entries": n, "batch": B, "reader_threads": threads,
                   "shuffle_buffer_entries": 16384, "skip_filter": "off", "parallelism": "single-gpu"},
        "host_stream_entries_per_s": host_rate,
        "cpu_baseline": None,
    }
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--reps", type=int, default=5,
                    help="timed repetitions of --steps steps per leg; the median is reported, with min and max")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--warmup-s", type=float, default=0.25,
                    help="warm-up also runs until this many seconds have passed (GPU clock ramp)")
    ap.add_argument("--workload", type=int, default=1)
    ap.add_argument("--bwd", choices=["sorted", "atomic"], default="sorted")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--graph", action=argparse.BooleanOptionalAction, default=True,
                    help="time the step as a captured HIP graph (default) or eagerly (--no-graph)")
    ap.add_argument("--composed", choices=sorted(COMPOSED), default=None,
                    help="time ComposedFeatureTransformer (fused vs reference composition) instead")
    ap.add_argument("--transform", choices=sorted(COMPOSED), default=None,
                    help="time the FT + post-FT epilogue (fused vs the reference ops) instead")
    ap.add_argument("--optimizer", action="store_true",
                    help="time the fused Ranger22 update of the FT parameters instead")
    ap.add_argument("--encode", choices=["halfka", "threats"], default=None,
                    help="time the GPU feature-index encoder instead")
    ap.add_argument("--export", action="store_true", help="time the GPU LEB128 encoder of the .nnue export instead")
    ap.add_argument("--pipeline", action="store_true",
                    help="time the host data pipeline with the copy to the GPU and the GPU encode instead")
    ap.add_argument("--configs", action=argparse.BooleanOptionalAction, default=True,
                    help="also time every workload (0-4) and list them under 'configs' (default on)")
    ap.add_argument("--traffic", choices=["live", "profile", "off"], default="live",
                    help="memory-side bytes per kernel: two rocprofv3 counter passes before the timing (live), "
                         "the committed profiles/traffic_<workload>.json (profile), or none")
    ap.add_argument("--zipf", type=float, default=None, metavar="ALPHA",
                    help="skewed feature frequencies (probability ~ 1 / (rank + 10)^ALPHA) instead of uniform ones; "
                         "a robustness run, not the headline")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build runs the FT on a single MI355X).", file=sys.stderr)
        return 2

    import torch

    from sft_amd import _native, workloads

    w = workloads.WORKLOADS[args.workload]
    special = args.composed or args.transform or args.optimizer or args.encode or args.export or args.pipeline
    # The counter passes run in child processes before this one touches the GPU.
    traffic = None
    if not special and args.zipf is None and args.traffic == "live":
        traffic = live_traffic(w.wid, log)
    if traffic is None and not special and args.zipf is None and args.traffic != "off":
        traffic = committed_traffic(w.name)
    dev = torch.device("cuda:0")
    _native.lib()  # fail loudly if the library is missing
    if args.composed:
        return bench_composed(args, dev)
    if args.transform:
        return bench_transform(args, dev)
    if args.optimizer:
        return bench_optimizer(args, dev)
    if args.encode:
        return bench_encode(args, dev)
    if args.export:
        return bench_export(args, dev)
    if args.pipeline:
        return bench_pipeline(args, dev)
    if w.quantized:
        return bench_q16(args, w, dev)

    l2 = l2_gather_ceiling(dev, args.warmup_s)
    log(f"[bench] L2-served 128-byte row gathers (probe): {l2['gbs']:.0f} GB/s; derived L2 peak "
        f"{L2_DERIVED_PEAK_GBS:.0f} GB/s")
    head, d = run_fp32(args, w, dev, zipf=args.zipf, traffic=traffic, l2_attainable=l2["gbs"], graph=args.graph,
                       hashes=True)
    ms = head["ms_per_step"]
    result = {
        "metric": METRIC,
        "value": w.B / (ms * 1e-3),
        "unit": "positions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup, "warmup_s": args.warmup_s,
        "ms_per_step": ms,
        "reps": head["reps"], "ms_per_step_min": head["ms_per_step_min"], "ms_per_step_max": head["ms_per_step_max"],
        "ms_per_step_reps": head["ms_per_step_reps"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic" if args.zipf is None else f"synthetic, Zipf-like feature frequencies (alpha {args.zipf})",
        "config": {
            "workload": w.name, "feature_set": w.feature_set, "batch": w.B, "num_inputs": w.N,
            "max_active": w.K, "active": [w.lo, w.hi], "output_size": w.L, "bwd": args.bwd,
            "feature_freq": "uniform" if args.zipf is None else f"1/(rank+10)^{args.zipf}",
            "launch": "hip_graph" if args.graph else "eager",
            "parallelism": "single-gpu",
            "input_sha256": head.pop("input_sha256"),
        },
        "eager_ms_per_step": head["eager_ms_per_step"],
        "step_bytes": head["step_bytes"],
        "step_gbs": head["step_gbs"],
        "step_compulsory_bytes": head["step_compulsory_bytes"],
        "step_compulsory_frac_of_hbm_peak": head["step_compulsory_frac_of_hbm_peak"],
        "step_traffic_bytes": head.get("step_traffic_bytes"),
        "step_traffic_frac_of_hbm_peak": head.get("step_traffic_frac_of_hbm_peak"),
        "roofline": head["roofline"],
        "l2_gather_ceiling": l2,
        "kernels": head["kernels"],
    }
    result["attainable"] = attainable(dev)
    log(f"[bench] attainable: 1 GiB device copy {result['attainable']['copy_gbs']:.0f} GB/s")
    if not args.no_cpu:
        log(f"[bench] cpu baseline ({args.cpu_seconds:.0f} s budget)")
        result["cpu_baseline"] = cpu_baseline(w, d, args.cpu_seconds)
        result["gpu_over_cpu"] = result["value"] / result["cpu_baseline"]["value"]
    else:
        result["cpu_baseline"] = None
    del d
    if args.configs and args.zipf is None:
        configs = []
        for wid in sorted(workloads.WORKLOADS):
            cw = workloads.WORKLOADS[wid]
            if wid == w.wid:
                entry = dict(head, workload=cw.name, dtype="fp32")
            elif cw.quantized:
                entry = run_q16(args, cw, dev, l2_attainable=l2["gbs"], traffic=committed_traffic(cw.name))
            else:
                entry, cd = run_fp32(args, cw, dev, traffic=committed_traffic(cw.name), l2_attainable=l2["gbs"],
                                     graph=args.graph)
                entry = dict(entry, workload=cw.name, dtype="fp32")
                if wid == 0 and not args.no_cpu:  # the CPU-runnable configuration: its own CPU baseline
                    log(f"[bench] cpu baseline of {cw.name} ({min(args.cpu_seconds, 8.0):.0f} s budget)")
                    entry["cpu_baseline"] = cpu_baseline(cw, cd, min(args.cpu_seconds, 8.0))
                    entry["gpu_over_cpu"] = entry["positions_per_s"] / entry["cpu_baseline"]["value"]
                del cd
            entry.pop("kernels", None)
            configs.append(entry)
            r = entry["roofline"]
            log(f"[bench] config {wid} {cw.name}: {entry['ms_per_step']:.3f} ms/step (median of {entry['reps']}), "
                f"{entry['positions_per_s'] / 1e6:.1f} M positions/s; {r['kernel']} hbm frac {r['frac']:.2f}, "
                f"logical {r['logical']['frac_of_hbm_peak']:.2f}")
            torch.cuda.empty_cache()
        result["configs"] = configs
        # Robustness, not the headline: the headline workload with Zipf-like
        # feature frequencies (real positions concentrate on a few features).
        skewed = []
        for alpha in (0.7, 1.0):
            entry, sd = run_fp32(args, w, dev, zipf=alpha, graph=args.graph)
            del sd
            skewed.append({"zipf_alpha": alpha, "feature_freq": f"1/(rank+10)^{alpha}",
                           "ms_per_step": entry["ms_per_step"], "positions_per_s": entry["positions_per_s"],
                           "bwd_tiled_gather_avg_ms": entry["kernels"].get("bwd_tiled_gather", {}).get("avg_ms")})
            log(f"[bench] {w.name} Zipf alpha {alpha}: {entry['ms_per_step']:.3f} ms/step")
            torch.cuda.empty_cache()
        result["skewed"] = skewed
        # The headline with the reference's own HalfKAv2_hm^ table height
        # (24 576 rows, FEAT/halfka_v2_hm.py:50) instead of 23 232, uniform rows.
        import dataclasses

        from src.model.modules.features.halfka_v2_hm import HalfKav2Hm

        wn = dataclasses.replace(w, name=w.name + "_n24576", N=HalfKav2Hm.NUM_INPUTS)
        entry, sd = run_fp32(args, wn, dev, graph=args.graph)
        del sd
        result["sensitivity"] = [{"num_inputs": wn.N, "ms_per_step": entry["ms_per_step"],
                                  "positions_per_s": entry["positions_per_s"],
                                  "fwd_f32_tiled_gather_avg_ms":
                                      entry["kernels"].get("fwd_f32_tiled_gather", {}).get("avg_ms"),
                                  "bwd_tiled_gather_avg_ms":
                                      entry["kernels"].get("bwd_tiled_gather", {}).get("avg_ms")}]
        log(f"[bench] {wn.name}: {entry['ms_per_step']:.3f} ms/step")
        torch.cuda.empty_cache()
        # The headline batch and width with index rows the GPU encoder makes
        # from random positions (HalfKAv2_hm: one king bucket's rows per
        # perspective, fewer active features than the uniform U[16, 32] rows)
        # over the encoder's 24 576-row table.
        try:
            entry, sd = run_fp32(args, w, dev, encoded=True, graph=args.graph)
        except (RuntimeError, ValueError, OSError) as e:  # a robustness leg: the line above stands without it
            log(f"[bench] encoder-rows leg failed: {e}")
            result["encoded"] = {"error": str(e)}
        else:
            del sd
            result["encoded"] = {"indices": "HalfKAv2_hm rows of the GPU encoder over random positions "
                                            "(sft_amd.positions.random_positions, seed 1)",
                                 "num_inputs": entry["num_inputs"],
                                 "active_mean": entry["active_mean"], "ms_per_step": entry["ms_per_step"],
                                 "positions_per_s": entry["positions_per_s"],
                                 "fwd_f32_tiled_gather_avg_ms":
                                     entry["kernels"].get("fwd_f32_tiled_gather", {}).get("avg_ms"),
                                 "bwd_tiled_gather_avg_ms":
                                     entry["kernels"].get("bwd_tiled_gather", {}).get("avg_ms")}
            log(f"[bench] {w.name} encoder rows ({entry['active_mean']:.1f} active): "
                f"{entry['ms_per_step']:.3f} ms/step")
        torch.cuda.empty_cache()
    print(json.dumps(result), flush=True)
    return 0


def run_fp32(args, w, dev, zipf=None, traffic=None, l2_attainable=None, graph=True, hashes=False, encoded=False):
    """Times the fp32 step of one workload (both perspectives through
    SparseLinearFunction, fwd + bwd); returns its measurements and the inputs."""
    import torch

    from sft_amd import _native, workloads
    from src.model.modules.feature_transformer import SparseLinearFunction
    from src.model.modules.feature_transformer import kernel as ftk

    if encoded:  # the encoder's HalfKAv2_hm rows index a table of HalfKav2Hm.NUM_INPUTS rows
        import dataclasses

        from src.model.modules.features.halfka_v2_hm import HalfKav2Hm

        w = dataclasses.replace(w, name=w.name + "_encoded", feature_set="HalfKAv2_hm", N=HalfKav2Hm.NUM_INPUTS)
    log(f"[bench] generating {w.name}: B={w.B} N={w.N} K={w.K} active U[{w.lo},{w.hi}] L={w.L}")
    d = workloads.make_fp32_inputs(w)
    if zipf is not None:
        log(f"[bench] Zipf-like feature frequencies, alpha={zipf}")
        d["idx_w"] = workloads.make_zipf_indices(workloads.rng(w.wid, workloads.S_WHITE), w.B, w.N, w.K, w.lo, w.hi,
                                                 zipf)
        d["idx_b"] = workloads.make_zipf_indices(workloads.rng(w.wid, workloads.S_BLACK), w.B, w.N, w.K, w.lo, w.hi,
                                                 zipf)
    if encoded:
        from sft_amd import encode, positions

        log(f"[bench] index rows from the GPU encoder over {w.B} random positions")
        boards, stm = positions.random_positions(w.B, seed=1)
        enc = encode.encode_batch(torch.from_numpy(boards).to(dev), torch.from_numpy(stm).to(dev), "HalfKAv2_hm")
        d["idx_w"] = enc["white"].cpu().numpy()
        d["idx_b"] = enc["black"].cpu().numpy()
        del enc
    iw = torch.from_numpy(d["idx_w"]).to(dev)
    ib = torch.from_numpy(d["idx_b"]).to(dev)
    W = torch.from_numpy(d["W"]).to(dev).requires_grad_(True)
    b = torch.from_numpy(d["bias"]).to(dev).requires_grad_(True)
    gw = torch.from_numpy(d["g_w"]).to(dev)
    gb = torch.from_numpy(d["g_b"]).to(dev)

    restore = None
    if args.bwd == "atomic":
        orig = ftk._BackwardKernel.__call__

        def atomic_call(self, *a, **k):
            k["atomic"] = True
            return orig(self, *a, **k)

        ftk._BackwardKernel.__call__ = atomic_call
        restore = orig

    def step():
        W.grad = None
        b.grad = None
        ow = SparseLinearFunction.apply(iw, W, b)
        ob = SparseLinearFunction.apply(ib, W, b)
        torch.autograd.backward([ow, ob], [gw, gb])

    nw = warm_up(step, args.warmup, args.warmup_s)
    log(f"[bench] warmup {nw} steps (at least {args.warmup} and {args.warmup_s} s)")

    # The eager step, then per-kernel durations from a second eager pass with the
    # library's launch events (which add ~0.1 ms per step of their own).
    eager = rep_stats(timed_reps(step, args.steps, args.reps))
    eager_ms = eager["ms_per_step"]
    log(f"[bench] eager {args.reps} x {args.steps} steps: {eager_ms:.3f} ms/step (median; "
        f"{eager['ms_per_step_min']:.3f}-{eager['ms_per_step_max']:.3f})")
    _native.prof_enable(True)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    prof = _native.prof_collect()
    _native.prof_enable(False)
    timing = eager
    if graph:
        # The whole step (both forwards, autograd backward, the grad sum) as one
        # HIP graph: the library makes no host synchronisation inside its calls.
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        warm_up(g.replay, args.warmup, args.warmup_s)
        timing = rep_stats(timed_reps(g.replay, args.steps, args.reps))
        log(f"[bench] graph {args.reps} x {args.steps} replays: {timing['ms_per_step']:.3f} ms/step (median; "
            f"{timing['ms_per_step_min']:.3f}-{timing['ms_per_step_max']:.3f})")
        del g
    ms = timing["ms_per_step"]
    if restore is not None:
        ftk._BackwardKernel.__call__ = restore

    step_bytes = workloads.step_bytes(d["idx_w"], d["idx_b"], w.N, w.L)
    kt = traffic["kind_step_bytes"] if traffic else {}
    kern = {}
    for kind, (tot, cnt) in prof.items():
        avg = tot / cnt
        lps = cnt / args.steps
        sb = kernel_step_bytes(kind, w, (d["idx_w"], d["idx_b"]))
        per_launch = sb / lps if sb else None
        kern[kind] = {"avg_ms": avg, "launches_per_step": lps, "bytes_per_launch": per_launch,
                      "gbs": (per_launch / (avg * 1e-3) / 1e9) if per_launch else None,
                      "traffic_per_launch": kt[kind] / lps if kind in kt else None}
        log(f"[bench]   {kind:22s} {avg:8.4f} ms x {lps:.0f}/step"
            + (f"  {kern[kind]['gbs']:8.1f} GB/s algorithmic" if per_launch else "")
            + (f"  {kern[kind]['traffic_per_launch'] / 1e6:7.1f} MB traffic" if kind in kt else ""))
    # the roofline's kernel: the one with the most time per step among those
    # with an algorithmic byte count (the sort and segment passes have none)
    dom = max((k for k in prof if kern[k]["bytes_per_launch"]), key=lambda k: prof[k][0])
    dk = kern[dom]
    compulsory = workloads.step_compulsory_bytes(w.B, w.K, w.N, w.L)
    out = {
        "feature_set": w.feature_set, "batch": w.B, "num_inputs": w.N, "max_active": w.K, "active": [w.lo, w.hi],
        "output_size": w.L, "step": "fwd + bwd of both perspectives through SparseLinearFunction",
        **timing, "eager_ms_per_step": eager_ms, "positions_per_s": w.B / (ms * 1e-3),
        "step_bytes": step_bytes, "step_gbs": step_bytes / (ms * 1e-3) / 1e9,
        "step_compulsory_bytes": compulsory,
        "step_compulsory_frac_of_hbm_peak": compulsory / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "roofline": roofline(dom, dk["bytes_per_launch"], dk["avg_ms"], dk["traffic_per_launch"],
                             traffic["source"] if traffic else None, l2_attainable),
        "kernels": kern,
    }
    if traffic:
        out["step_traffic_bytes"] = traffic["step_bytes"]
        out["step_traffic_frac_of_hbm_peak"] = traffic["step_bytes"] / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS
        out["traffic_source"] = traffic["source"]
    if hashes:
        out["input_sha256"] = {k: workloads.sha256(v) for k, v in d.items()}
    out["active_mean"] = float(((d["idx_w"] >= 0).sum() + (d["idx_b"] >= 0).sum()) / (2 * w.B))
    return out, d


if __name__ == "__main__":
    sys.exit(main())
