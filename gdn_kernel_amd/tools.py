"""Developer tools around one FlashInfer-Trace workload: sanitizer-style checks
and a rocprofv3 wrapper.

The reference's harness offers ``flashinfer_bench_run_sanitizer(solution,
workload, sanitizer_types=["memcheck", "racecheck", "synccheck", "initcheck"])``
and ``flashinfer_bench_run_ncu(solution, workload, set=..., page=...)``
(/root/reference/README.md:187-214), both NVIDIA tools.  On MI355X the
equivalents are built here:

* ``run_sanitizer`` -- functional checks of this library's kernels on one
  workload, run through the same destination-passing entry points:
    - ``initcheck``: every output element is written (outputs are pre-filled
      with two different sentinels in two runs; an element still holding its
      sentinel in both is unwritten);
    - ``memcheck``: every input and output lives inside a larger allocation with
      guard bytes on both sides; after the launch the guards must be intact
      (no out-of-bounds writes) and the inputs unchanged (no writes to inputs);
    - ``racecheck`` / ``synccheck``: repeated launches on identical inputs must
      give bit-identical outputs (a missing wait or a race between waves shows
      up as run-to-run differences).
  GPU AddressSanitizer builds are not used: they need an xnack+ code object,
  which this build does not make.
* ``run_profiler`` -- runs the workload in a child process under ``rocprofv3``
  (``--kernel-trace --stats``, or ``--pmc <counters>`` in a run of its own) and
  returns a text summary of this library's kernels from the CSV output.

Usage:
  python -m gdn_kernel_amd.tools sanitize --dataset ROOT --definition NAME [--workload UUID]
  python -m gdn_kernel_amd.tools profile  --dataset ROOT --definition NAME [--workload UUID]
         [--pmc COUNTER ...] [--iterations N] [--out DIR]
"""
from __future__ import annotations

import argparse
import csv
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

import torch

from . import bench_runner as br

__all__ = ["run_sanitizer", "run_profiler", "SANITIZERS"]

SANITIZERS = ("initcheck", "memcheck", "racecheck", "synccheck")
GUARD_BYTES = 4096
_GUARD = 0xA5


def _pick(ts: br.TraceSet, definition: str, workload: str | None):
    if definition not in ts.definitions:
        raise ValueError(f"Definition '{definition}' not found in trace set")
    wls = ts.workloads.get(definition, [])
    if workload is not None:
        wls = [w for w in wls if w.uuid == workload]
    if not wls:
        raise ValueError(f"no workload {workload or ''} for {definition}")
    return ts.definitions[definition], wls[0]


def _guarded_like(t: torch.Tensor):
    """(view, backing) -- a copy of ``t`` placed between two guard regions of a
    larger uint8 allocation on the same device (the view keeps 256-byte alignment)."""
    nbytes = t.numel() * t.element_size()
    backing = torch.full((GUARD_BYTES + nbytes + GUARD_BYTES,), _GUARD, dtype=torch.uint8,
                         device=t.device)
    inner = backing[GUARD_BYTES:GUARD_BYTES + nbytes].view(t.dtype).view(t.shape)
    inner.copy_(t)
    return inner, backing


def _guards_intact(backing: torch.Tensor, nbytes: int) -> bool:
    lo, hi = backing[:GUARD_BYTES], backing[GUARD_BYTES + nbytes:]
    return bool((lo == _GUARD).all()) and bool((hi == _GUARD).all())


def run_sanitizer(root, definition: str, workload: str | None = None,
                  sanitizer_types=("initcheck", "memcheck", "racecheck"), device=None,
                  repeats: int = 3) -> str:
    """Run the selected checks on one workload; returns a report whose last line is
    ``SANITIZER SUMMARY: <n> error(s)``."""
    for s in sanitizer_types:
        if s not in SANITIZERS:
            raise ValueError(f"unknown sanitizer {s!r} (known: {', '.join(SANITIZERS)})")
    if device is None:
        if not torch.cuda.is_available():
            raise RuntimeError("the sanitizer checks need a ROCm GPU")
        device = torch.device("cuda", torch.cuda.current_device())
    ts = br.TraceSet.from_path(root)
    defn, wl = _pick(ts, definition, workload)
    sol = br.solution_for(defn)
    if sol is None:
        raise ValueError(f"{definition} is not implemented by this library")
    kernel, _, in_names = sol
    ins = br.materialize_inputs(defn, wl, root, device)
    axes = br.resolve_axes(defn, wl)
    lines, errors = [f"== {definition} / workload {wl.uuid}"], 0

    def launch(inputs, outputs):
        kernel(*[inputs[n] for n in in_names], *[outputs[n] for n in br._OUT])
        torch.cuda.synchronize()

    if "initcheck" in sanitizer_types:
        runs = []
        for fill in (float("nan"), 1.0e30):
            outs = br.allocate_outputs(defn, axes, device, fill=fill)
            launch(ins, outs)
            runs.append((fill, outs))
        bad = 0
        for name in br._OUT:
            o0, o1 = runs[0][1][name], runs[1][1][name]
            sentinel = torch.tensor(runs[1][0], dtype=o1.dtype, device=o1.device)
            unwritten = torch.isnan(o0) & (o1 == sentinel)
            bad += int(unwritten.sum())
            if unwritten.any():
                lines.append(f"initcheck: {int(unwritten.sum())} element(s) of {name} never written")
        lines.append(f"initcheck: {'FAILED' if bad else 'PASSED'}")
        errors += bool(bad)

    if "memcheck" in sanitizer_types:
        g_ins, backs = {}, {}
        for n, t in ins.items():
            if torch.is_tensor(t):
                g_ins[n], backs[n] = _guarded_like(t)
            else:
                g_ins[n] = t
        plain = br.allocate_outputs(defn, axes, device)
        g_outs = {}
        for n, t in plain.items():
            g_outs[n], backs["out:" + n] = _guarded_like(t)
        launch(g_ins, g_outs)
        bad = []
        for key, back in backs.items():
            t = g_outs[key[4:]] if key.startswith("out:") else g_ins[key]
            if not _guards_intact(back, t.numel() * t.element_size()):
                bad.append(f"write outside {key}")
        for n, t in ins.items():
            if torch.is_tensor(t) and not torch.equal(g_ins[n], t):
                bad.append(f"input {n} modified")
        for b in bad:
            lines.append(f"memcheck: {b}")
        lines.append(f"memcheck: {'FAILED' if bad else 'PASSED'}")
        errors += bool(bad)

    if "racecheck" in sanitizer_types or "synccheck" in sanitizer_types:
        first, diffs = None, 0
        for _ in range(max(2, repeats)):
            outs = br.allocate_outputs(defn, axes, device)
            launch(ins, outs)
            cur = {n: outs[n].clone() for n in br._OUT}
            if first is None:
                first = cur
            else:
                for n in br._OUT:
                    same = (cur[n] == first[n]) | (torch.isnan(cur[n]) & torch.isnan(first[n]))
                    diffs += int((~same).sum())
        name = "racecheck" if "racecheck" in sanitizer_types else "synccheck"
        if diffs:
            lines.append(f"{name}: {diffs} element(s) differ between identical launches")
        lines.append(f"{name}: {'FAILED' if diffs else 'PASSED'}")
        errors += bool(diffs)

    lines.append(f"SANITIZER SUMMARY: {errors} error(s)")
    return "\n".join(lines)


def _rocprofv3() -> str:
    for cand in (shutil.which("rocprofv3"), "/opt/rocm/bin/rocprofv3"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("rocprofv3 not found")


def run_profiler(root, definition: str, workload: str | None = None, pmc=None,
                 iterations: int = 20, out_dir=None, timeout: int = 300) -> str:
    """Profile one workload with rocprofv3 in a child process.  Without ``pmc``:
    kernel trace and per-kernel statistics; with ``pmc``: those counters (one
    run; rocprofv3 does not split counters over passes, so keep each hardware
    block within its limits).  Returns a text summary of this library's kernels."""
    root = Path(root).resolve()
    ts = br.TraceSet.from_path(root)
    defn, wl = _pick(ts, definition, workload)
    out = Path(out_dir) if out_dir else Path(tempfile.mkdtemp(prefix="gdn_prof_"))
    out.mkdir(parents=True, exist_ok=True)
    cmd = [_rocprofv3()]
    cmd += ["--pmc", *pmc] if pmc else ["--kernel-trace", "--stats"]
    cmd += ["--output-format", "csv", "-d", str(out), "-o", "run", "--",
            sys.executable, "-m", "gdn_kernel_amd.tools", "run-workload", "--dataset", str(root),
            "--definition", defn.name, "--workload", wl.uuid, "--iterations", str(iterations)]
    env = dict(os.environ)
    pkg_root = str(Path(__file__).resolve().parent.parent)
    env["PYTHONPATH"] = pkg_root + os.pathsep + env.get("PYTHONPATH", "")
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout, env=env,
                         cwd=tempfile.gettempdir())
    csvs = sorted(out.rglob("run_counter_collection.csv" if pmc else "run_kernel_stats.csv"))
    if not csvs:
        raise RuntimeError(f"rocprofv3 wrote no results (exit {res.returncode}):\n"
                           + (res.stdout + res.stderr)[-2000:])
    rows = list(csv.DictReader(open(csvs[0])))
    lines = [f"== rocprofv3 {'--pmc ' + ' '.join(pmc) if pmc else '--kernel-trace --stats'}: "
             f"{defn.name} / {wl.uuid}, {iterations} launches ({csvs[0]})"]
    if pmc:
        agg: dict = {}
        for r in rows:
            if "gdn" not in r["Kernel_Name"]:
                continue
            k = r["Kernel_Name"].split("(")[0]
            d = agg.setdefault(k, {"_dispatch": set()})
            d["_dispatch"].add(r["Dispatch_Id"])
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        for k, d in agg.items():
            n = len(d.pop("_dispatch"))
            lines.append(f"{k} ({n} dispatches, mean per dispatch):")
            lines += [f"  {c} = {v / n:,.0f}" for c, v in sorted(d.items())]
    else:
        lines.append(f"{'kernel':<70} {'calls':>6} {'avg us':>10} {'min us':>10} {'max us':>10}")
        for r in rows:
            if "gdn" not in r["Name"]:
                continue
            lines.append(f"{r['Name'].split('(')[0][:70]:<70} {int(r['Calls']):>6} "
                         f"{float(r['AverageNs']) / 1e3:>10.2f} {float(r['MinNs']) / 1e3:>10.2f} "
                         f"{float(r['MaxNs']) / 1e3:>10.2f}")
    return "\n".join(lines)


def _run_workload_child(root, definition, workload, iterations: int) -> int:
    """The profiled program: launch one workload's kernel ``iterations`` times."""
    ts = br.TraceSet.from_path(root)
    defn, wl = _pick(ts, definition, workload)
    kernel, _, in_names = br.solution_for(defn)
    device = torch.device("cuda", torch.cuda.current_device())
    ins = br.materialize_inputs(defn, wl, root, device)
    outs = br.allocate_outputs(defn, br.resolve_axes(defn, wl), device)
    args = [ins[n] for n in in_names] + [outs[n] for n in br._OUT]
    for _ in range(iterations):
        kernel(*args)
    torch.cuda.synchronize()
    return 0


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="sanitizer checks and rocprofv3 profiles of one workload")
    ap.add_argument("command", choices=["sanitize", "profile", "run-workload"])
    ap.add_argument("--dataset", default=os.environ.get("FIB_DATASET_PATH"))
    ap.add_argument("--definition", required=True)
    ap.add_argument("--workload")
    ap.add_argument("--sanitizers", nargs="+", default=["initcheck", "memcheck", "racecheck"])
    ap.add_argument("--pmc", nargs="+")
    ap.add_argument("--iterations", type=int, default=20)
    ap.add_argument("--out")
    args = ap.parse_args(argv)
    if not args.dataset:
        print("FIB_DATASET_PATH is not set and no --dataset given", file=sys.stderr)
        return 2
    if args.command == "run-workload":
        return _run_workload_child(args.dataset, args.definition, args.workload, args.iterations)
    if args.command == "sanitize":
        rep = run_sanitizer(args.dataset, args.definition, args.workload, tuple(args.sanitizers))
        print(rep)
        return 0 if rep.endswith(" 0 error(s)") else 1
    print(run_profiler(args.dataset, args.definition, args.workload, args.pmc, args.iterations,
                       args.out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
