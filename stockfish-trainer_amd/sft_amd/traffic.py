"""Memory-side traffic per kernel dispatch from two rocprofv3 counter passes.

Each pass is its own child process running `sft_amd/profile_step.py` (a few FT
steps of one workload, then a 1 GiB calibration copy) under

  rocprofv3 --pmc FETCH_SIZE TCC_HIT_sum ...
  rocprofv3 --pmc WRITE_SIZE TCC_MISS_sum TCC_EA0_RDREQ_DRAM_sum ...

FETCH_SIZE and WRITE_SIZE count the L2's requests to the memory side (the
data fabric), so they include lines the 256 MB MALL serves as well as HBM
accesses: an upper bound of the HBM bytes.  Each is scaled by the ratio of the
calibration copy's true bytes (1 GiB read, 1 GiB written) to what the same
counter reads for it.  The caller must not have initialised the GPU in its own
process when it starts the passes (a profiled child of a process holding the
GPU is not allowed on the target machines).

  python stockfish-trainer_amd/sft_amd/traffic.py --workload 1 --dir /tmp/sft_pmc \
      --md profiles/pmc_traffic_halfka_b65536.md
"""

from __future__ import annotations

import argparse
import collections
import csv
import glob
import os
import re
import shutil
import subprocess
import sys
import tempfile

PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ROOT = os.path.dirname(PKG)
PROFILE_STEP = os.path.join(PKG, "sft_amd", "profile_step.py")
CALIB_KIB = 1 << 20  # the calibration copy: 1 GiB read and 1 GiB written
PASS_A = ["FETCH_SIZE", "TCC_HIT_sum"]
PASS_B = ["WRITE_SIZE", "TCC_MISS_sum", "TCC_EA0_RDREQ_DRAM_sum"]

# kernel-name pattern -> the library's timing kind of that kernel (sft_prof_kind_name)
KINDS = [
    (r"\bfwd_tiled_kernel<", "fwd_f32_tiled_gather"),
    (r"\bfwd_f32_kernel<", "fwd_f32_gather"),
    (r"\btile_relayout_kernel\b", "fwd_tile_relayout"),
    (r"\brelayout_rank_kernel\b", "fwd_tile_relayout"),  # the re-layout with the staged rank lists
    (r"\bfold_relayout_kernel\b", "fwd_fold_relayout"),
    (r"\bfwd_i16_tiled_kernel\b", "fwd_i16_tiled_gather"),
    (r"\bfwd_i16_ranked_kernel\b", "fwd_i16_tiled_gather"),
    (r"\brank_lists_kernel\b", "fwd_rank_lists"),
    (r"\brank_lists_wide_kernel<", "fwd_rank_lists"),
    (r"\bi16_relayout_kernel\b", "fwd_tile_relayout"),
    (r"\bfwd_i16_kernel<", "fwd_i16_gather"),
    (r"\bbwd_tiled_gather_kernel<", "bwd_tiled_gather"),
    (r"\bgather_rows_kernel<", "bwd_feature_gather"),
    (r"\bbias_partial_kernel<", "bwd_bias_partial"),
    (r"\bbias_final_kernel<", "bwd_bias_final"),
    (r"\bseg_offsets_kernel\b", "bwd_segment_offsets"),
    (r"\bradix_", "bwd_feature_sort"),
    (r"\bbucket_sort_kernel<", "bwd_feature_sort"),
    (r"\bzero_kernel\b", "bwd_zero_fill"),
    (r"\bscatter_atomic_kernel<", "bwd_atomic_scatter"),
    (r"\bvirtual_reduce_kernel\b", "bwd_virtual_reduce"),
    (r"\bbwd_epilogue_kernel\b", "bwd_epilogue"),
]


def short_name(name: str) -> str:
    n = name.replace("(anonymous namespace)::", "").replace("sft::", "").replace("void ", "")
    n = re.sub(r"\(.*", "", n)
    return n[:60]


def kind_of(name: str) -> str | None:
    for pat, kind in KINDS:
        if re.search(pat, name):
            return kind
    return None


def _run_pass(counters, workload: int, steps: int, out_dir: str, timeout: float, log) -> str:
    exe = shutil.which("rocprofv3")
    if exe is None:
        raise RuntimeError("rocprofv3 not found")
    shutil.rmtree(out_dir, ignore_errors=True)
    cmd = [exe, "--pmc", *counters, "-d", out_dir, "-o", "p", "--output-format", "csv", "--",
           sys.executable, PROFILE_STEP, "--workload", str(workload), "--steps", str(steps)]
    env = dict(os.environ, TMPDIR="/tmp")
    log("[traffic] " + " ".join(["rocprofv3", "--pmc", *counters, "--", "python",
                                 os.path.relpath(PROFILE_STEP, ROOT), "--workload", str(workload)]))
    r = subprocess.run(cmd, cwd=ROOT, env=env, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, timeout=timeout,
                       text=True)
    found = glob.glob(os.path.join(out_dir, "**", "*counter_collection.csv"), recursive=True)
    if not found:
        tail = "\n".join(r.stdout.splitlines()[-5:])
        raise RuntimeError(f"rocprofv3 pass {counters} left no counter file (rc {r.returncode}): {tail}")
    # rocprofv3 may end with a fault of its own after the program finished and the
    # files are complete; the program's last line says whether it did finish.
    if "[profile] done" not in r.stdout:
        raise RuntimeError(f"profiled program did not finish (rc {r.returncode})")
    return found[0]


def _read(path: str):
    per = collections.defaultdict(lambda: collections.defaultdict(list))
    with open(path) as f:
        for row in csv.DictReader(f):
            per[row["Kernel_Name"]][row["Counter_Name"]].append(float(row["Counter_Value"]))
    return per


def measure(workload: int, out_dir: str, steps: int = 3, timeout: float = 120.0, log=print) -> dict:
    """Runs both counter passes over `steps + 1` FT steps of `workload`; returns
    {"kernels": {name: {...}}, "kind_step_bytes": {kind: bytes per step}, "step_bytes",
    "fetch_scale", "write_scale", "commands"}."""
    pa = _run_pass(PASS_A, workload, steps, os.path.join(out_dir, "pmcA"), timeout, log)
    pb = _run_pass(PASS_B, workload, steps, os.path.join(out_dir, "pmcB"), timeout, log)
    A, Bc = _read(pa), _read(pb)
    calib = [k for k in A if k.startswith("__amd_rocclr_copyBuffer")]
    cf = max(v for k in calib for v in A[k]["FETCH_SIZE"])
    cw = max(v for k in [k for k in Bc if k.startswith("__amd_rocclr_copyBuffer")] for v in Bc[k]["WRITE_SIZE"])
    fscale, wscale = CALIB_KIB / cf, CALIB_KIB / cw
    kernels, kinds = {}, {}  # kinds: bytes per step of each timing kind
    step_total = 0.0
    for k in A:
        if k.startswith("__amd") or "FillFunctor" in k or k not in Bc:
            continue  # the calibration copy and the fill of its source buffer
        fetch = [v * fscale * 1024 for v in A[k]["FETCH_SIZE"]]
        write = [v * wscale * 1024 for v in Bc[k]["WRITE_SIZE"]]
        hit, miss = sum(A[k]["TCC_HIT_sum"]), sum(Bc[k]["TCC_MISS_sum"])
        rd = Bc[k]["TCC_EA0_RDREQ_DRAM_sum"]
        e = {"short": short_name(k), "kind": kind_of(k), "dispatches": len(fetch),
             "fetch_bytes": sum(fetch) / len(fetch), "write_bytes": sum(write) / len(write),
             "l2_hit": hit / (hit + miss) if hit + miss else None, "ea_read_requests": sum(rd) / len(rd)}
        kernels[k] = e
        step_total += sum(fetch) + sum(write)
        if e["kind"] is not None:  # a kind may span several kernels (the sort's passes)
            kinds[e["kind"]] = kinds.get(e["kind"], 0.0) + (sum(fetch) + sum(write)) / (steps + 1)
    prog = f"python {os.path.relpath(PROFILE_STEP, ROOT)} --workload {workload} --steps {steps}"
    return {"kernels": kernels, "kind_step_bytes": kinds, "step_bytes": step_total / (steps + 1),
            "fetch_scale": fscale, "write_scale": wscale, "calib_fetch_kib": cf, "calib_write_kib": cw,
            "commands": [f"rocprofv3 --pmc {' '.join(PASS_A)} -d <dir>/pmcA -o p --output-format csv -- {prog}",
                         f"rocprofv3 --pmc {' '.join(PASS_B)} -d <dir>/pmcB -o p --output-format csv -- {prog}"]}


def summary_md(t: dict, title: str) -> str:
    lines = [f"# Memory-side traffic per dispatch — {title}", "",
             "Two counter passes, each its own run (repo root on the MI355X box; run by",
             "`stockfish-trainer_amd/sft_amd/traffic.py` and by `bench.py`):", "", "```", *t["commands"], "```", "",
             f"Calibration (1 GiB device copy): FETCH_SIZE = {t['calib_fetch_kib']:.0f} KiB, WRITE_SIZE = "
             f"{t['calib_write_kib']:.0f} KiB, so FETCH_SIZE is scaled by {t['fetch_scale']:.3f} and WRITE_SIZE by "
             f"{t['write_scale']:.3f}.  Both count L2 requests to the memory side, MALL hits included.",
             f"Whole step (every kernel, both perspectives): {t['step_bytes'] / 1e9:.3f} GB.", "",
             "| kernel | dispatches | fetch MB | write MB | L2 hit % | EA read req (M) |", "|---|---|---|---|---|---|"]
    for e in t["kernels"].values():
        hit = "" if e["l2_hit"] is None else f"{100 * e['l2_hit']:.0f}"
        lines.append(f"| `{e['short']}` | {e['dispatches']} | {e['fetch_bytes'] / 1e6:.1f} | "
                     f"{e['write_bytes'] / 1e6:.1f} | {hit} | {e['ea_read_requests'] / 1e6:.2f} |")
    return "\n".join(lines) + "\n"


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--dir", default=None, help="where rocprofv3 writes its passes (default: a new temporary directory)")
    ap.add_argument("--md", default=None, help="write the summary table to this file")
    ap.add_argument("--json", default=None, help="write the per-kind bytes per step (bench.py reads it) here")
    ap.add_argument("--title", default=None)
    args = ap.parse_args()
    sys.path.insert(0, PKG)
    from sft_amd import workloads

    out_dir = args.dir or tempfile.mkdtemp(prefix="sft_pmc_")
    t = measure(args.workload, out_dir, args.steps)
    text = summary_md(t, args.title or workloads.WORKLOADS[args.workload].name)
    if args.md:
        with open(args.md, "w") as f:
            f.write(text)
    if args.json:
        import json

        keep = {k: t[k] for k in ("kind_step_bytes", "step_bytes", "fetch_scale", "write_scale", "commands")}
        keep["workload"] = workloads.WORKLOADS[args.workload].name
        with open(args.json, "w") as f:
            json.dump(keep, f, indent=1)
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
