"""Offline FlashInfer-Trace runner for the GDN definitions.

The reference evaluates its kernels with the FlashInfer-Bench harness
(/root/reference/scripts/run_local.py:30-76): it loads a TraceSet (definitions,
workloads) from ``$FIB_DATASET_PATH``, runs the solution on every workload of
its definition with ``BenchmarkConfig(warmup_runs=3, iterations=100,
num_trials=5)`` and reports, per workload uuid, ``status``, ``latency_ms``,
``reference_latency_ms``, ``speedup_factor``, ``max_abs_error`` and
``max_rel_error`` (run_local.py:60-76, printed as in :79-101).  The harness and
the contest dataset are not installed here, so this module reads the same
on-disk FlashInfer-Trace layout itself and runs this library's kernels:

* definitions: ``<root>/definitions/**/<name>.json`` -- ``name``, ``op_type``,
  ``axes`` ({axis: {"type": "const", "value": n} | {"type": "var"}}),
  ``inputs`` / ``outputs`` ({name: {"shape": [axis | int, ...] | null,
  "dtype": "bfloat16" | "float32" | ...}}, in call order), optional
  ``reference`` (Python source defining ``run``);
* workloads: ``<root>/workloads/**/*.jsonl``, one JSON object per line:
  ``{"definition": name, "workload": {"uuid", "axes": {axis: n},
  "inputs": {name: {"type": "random"} | {"type": "scalar", "value": x} |
  {"type": "safetensors", "path": rel, "tensor_key": key}}}}`` (a bare
  workload object with a ``definition`` field is accepted too).

Definitions whose name starts with ``gdn_decode`` or ``gdn_prefill`` run on
``gdn_kernel_amd.decode.kernel`` / ``gdn_kernel_amd.prefill.kernel``, called in
destination-passing style with the definition's input and output tensors
(README.md:227-233).  Ground truth and ``reference_latency_ms`` come from the
float32 PyTorch implementations in ``gdn_kernel_amd.reference``, or, with
``use_definition_reference``, from executing the definition's own ``reference``
source (which is what the harness does; only do that for a dataset you trust).

Usage: python -m gdn_kernel_amd.bench_runner [--dataset PATH] [--definition NAME]
       [--warmup 3] [--iterations 100] [--trials 5] [--json OUT]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import statistics
import sys
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Optional

import torch

__all__ = ["Definition", "Workload", "TraceSet", "BenchmarkConfig", "resolve_axes",
           "materialize_inputs", "allocate_outputs", "run_workload", "run_benchmark",
           "print_results", "make_definition", "write_trace_set", "SOLUTION_NAME"]

SOLUTION_NAME = "gdn-mi355x-hip"

_DTYPES = {
    "bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32,
    "float64": torch.float64, "int32": torch.int32, "int64": torch.int64,
    "int8": torch.int8, "uint8": torch.uint8, "bool": torch.bool,
}


def torch_dtype(name: str) -> torch.dtype:
    try:
        return _DTYPES[name]
    except KeyError:
        raise ValueError(f"unsupported dtype {name!r}") from None


@dataclass
class Definition:
    name: str
    op_type: str
    axes: dict
    inputs: dict          # name -> {"shape": [...] | None, "dtype": str}, call order
    outputs: dict
    reference: Optional[str] = None
    raw: dict = field(default_factory=dict, repr=False)

    @classmethod
    def from_json(cls, d: dict) -> "Definition":
        for key in ("name", "axes", "inputs", "outputs"):
            if key not in d:
                raise ValueError(f"definition is missing {key!r}")
        return cls(name=d["name"], op_type=d.get("op_type", ""), axes=d["axes"],
                   inputs=d["inputs"], outputs=d["outputs"], reference=d.get("reference"),
                   raw=d)


@dataclass
class Workload:
    definition: str
    uuid: str
    axes: dict
    inputs: dict

    @classmethod
    def from_json(cls, d: dict) -> "Workload":
        body = d.get("workload", d)
        name = d.get("definition", body.get("definition"))
        if not name:
            raise ValueError("workload names no definition")
        if "uuid" not in body:
            raise ValueError(f"workload of {name} has no uuid")
        return cls(definition=name, uuid=str(body["uuid"]), axes=dict(body.get("axes", {})),
                   inputs=dict(body.get("inputs", {})))


@dataclass
class TraceSet:
    root: Path
    definitions: dict
    workloads: dict

    @classmethod
    def from_path(cls, root) -> "TraceSet":
        root = Path(root)
        if not root.is_dir():
            raise FileNotFoundError(f"trace set root {root} is not a directory")
        defs, wls = {}, {}
        for path in sorted((root / "definitions").rglob("*.json")):
            d = Definition.from_json(json.loads(path.read_text()))
            defs[d.name] = d
        for path in sorted((root / "workloads").rglob("*.jsonl")):
            for ln, line in enumerate(path.read_text().splitlines(), 1):
                if not line.strip():
                    continue
                try:
                    w = Workload.from_json(json.loads(line))
                except (ValueError, json.JSONDecodeError) as exc:
                    raise ValueError(f"{path}:{ln}: {exc}") from None
                wls.setdefault(w.definition, []).append(w)
        return cls(root=root, definitions=defs, workloads=wls)


@dataclass
class BenchmarkConfig:
    """Timing and tolerance settings; the timing defaults are run_local.py:33's."""
    warmup_runs: int = 3
    iterations: int = 100
    num_trials: int = 5
    reference_iterations: int = 3
    # (rtol, atol) per output name; other outputs use `default_tol`.
    tolerances: dict = field(default_factory=lambda: {"output": (1e-2, 1e-2),
                                                      "new_state": (1e-3, 1e-5)})
    default_tol: tuple = (1e-2, 1e-2)
    use_definition_reference: bool = False


def resolve_axes(defn: Definition, wl: Workload) -> dict:
    """Axis values: constants from the definition, variables from the workload."""
    out = {}
    for name, spec in defn.axes.items():
        kind = spec.get("type", "const") if isinstance(spec, dict) else "const"
        if kind == "const":
            out[name] = int(spec["value"] if isinstance(spec, dict) else spec)
        elif name in wl.axes:
            out[name] = int(wl.axes[name])
        else:
            raise ValueError(f"workload {wl.uuid} gives no value for axis {name!r} of {defn.name}")
    extra = set(wl.axes) - set(defn.axes)
    if extra:
        raise ValueError(f"workload {wl.uuid} sets unknown axes {sorted(extra)}")
    return out


def _shape(spec: dict, axes: dict, what: str) -> Optional[tuple]:
    shape = spec.get("shape")
    if shape is None:
        return None
    dims = []
    for d in shape:
        if isinstance(d, int):
            dims.append(d)
        elif d in axes:
            dims.append(axes[d])
        else:
            raise ValueError(f"{what}: unknown axis {d!r}")
    return tuple(dims)


def _seed(uuid: str, name: str) -> int:
    return int.from_bytes(hashlib.sha256(f"{uuid}/{name}".encode()).digest()[:8], "little") >> 1


def materialize_inputs(defn: Definition, wl: Workload, root, device) -> dict:
    """Input tensors (or Python scalars) of one workload, on ``device``."""
    axes = resolve_axes(defn, wl)
    out = {}
    blobs = {}
    for name, spec in defn.inputs.items():
        shape = _shape(spec, axes, f"{defn.name}.{name}")
        dtype = torch_dtype(spec["dtype"])
        src = wl.inputs.get(name, {"type": "random"})
        kind = src.get("type", "random")
        if kind == "scalar":
            val = src["value"]
            out[name] = (val if shape in (None, ()) else
                         torch.full(shape, val, dtype=dtype, device=device))
        elif kind == "safetensors":
            from safetensors.torch import load_file  # loads tensors only; executes nothing
            path = (Path(root) / src["path"]).resolve()
            if path not in blobs:
                blobs[path] = load_file(str(path))
            key = src.get("tensor_key", name)
            if key not in blobs[path]:
                raise ValueError(f"{path} has no tensor {key!r}")
            t = blobs[path][key]
            if shape is not None and tuple(t.shape) != shape:
                raise ValueError(f"{defn.name}.{name}: blob shape {tuple(t.shape)} != {shape}")
            out[name] = t.to(device=device, dtype=dtype).contiguous()
        elif kind == "random":
            gen = torch.Generator(device="cpu")
            gen.manual_seed(_seed(wl.uuid, name))
            if shape is None:
                out[name] = float(torch.randn((), generator=gen))
            elif dtype.is_floating_point:
                out[name] = torch.randn(shape, generator=gen).to(device=device, dtype=dtype)
            else:
                raise ValueError(f"{defn.name}.{name}: random integer inputs are not generated "
                                 "(give them as safetensors or scalars)")
        else:
            raise ValueError(f"{defn.name}.{name}: unknown input type {kind!r}")
    return out


def allocate_outputs(defn: Definition, axes: dict, device, fill=float("nan")) -> dict:
    """Destination tensors of the definition's outputs (NaN-filled floats)."""
    out = {}
    for name, spec in defn.outputs.items():
        shape = _shape(spec, axes, f"{defn.name}.{name}")
        dtype = torch_dtype(spec["dtype"])
        t = torch.empty(shape or (), dtype=dtype, device=device)
        if dtype.is_floating_point:
            t.fill_(fill)
        out[name] = t
    return out


# Parameter order of this library's entry points (the reference's DPS signatures,
# kernel.cu:101-113 and kernel_prefill.cu:300-306).
_DECODE_IN = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "scale")
_PREFILL_IN = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens", "scale")
_OUT = ("output", "new_state")


def solution_for(defn: Definition):
    """(kernel, reference, input names) for a supported definition, else None."""
    from . import reference as R
    from .binding import decode_kernel, prefill_kernel
    if defn.name.startswith("gdn_decode"):
        return decode_kernel, R.decode_reference, _DECODE_IN
    if defn.name.startswith("gdn_prefill"):
        return prefill_kernel, R.prefill_reference, _PREFILL_IN
    return None


def _definition_reference(defn: Definition) -> Callable:
    ns: dict = {}
    exec(compile(defn.reference, f"<reference of {defn.name}>", "exec"), ns)  # noqa: S102
    if "run" not in ns:
        raise ValueError(f"the reference of {defn.name} defines no run()")
    return ns["run"]


def _time_ms(fn, warmup: int, iterations: int, trials: int) -> float:
    """Median over trials of the mean per-call time (HIP events on the current stream)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    per_trial = []
    for _ in range(trials):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(iterations):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        per_trial.append(e0.elapsed_time(e1) / iterations)
    return statistics.median(per_trial)


def _errors(got: torch.Tensor, ref: torch.Tensor):
    g, r = got.double(), ref.double()
    diff = (g - r).abs()
    if diff.numel() == 0:
        return 0.0, 0.0
    max_abs = float(diff.max())
    max_rel = float((diff / r.abs().clamp_min(1e-12)).max())
    return max_abs, max_rel


def run_workload(defn: Definition, wl: Workload, root, cfg: BenchmarkConfig, device) -> dict:
    """Evaluate one workload; returns run_local.py's per-workload entry."""
    entry = {"status": "RUNTIME_ERROR", "solution": SOLUTION_NAME}
    sol = solution_for(defn)
    if sol is None:
        entry["status"] = "UNSUPPORTED_DEFINITION"
        return entry
    kernel, reference, in_names = sol
    try:
        ins = materialize_inputs(defn, wl, root, device)
        axes = resolve_axes(defn, wl)
        missing = [n for n in in_names if n not in ins] + [n for n in _OUT if n not in defn.outputs]
        if missing:
            entry["status"] = "UNSUPPORTED_DEFINITION"
            entry["error"] = f"definition lacks {missing}"
            return entry
        outs = allocate_outputs(defn, axes, device)
        args = [ins[n] for n in in_names] + [outs[n] for n in _OUT]
        kernel(*args)
        torch.cuda.synchronize()
        if cfg.use_definition_reference and defn.reference:
            ref_fn = _definition_reference(defn)
            ref_call = lambda: ref_fn(**{n: ins[n] for n in defn.inputs})  # noqa: E731
        else:
            ref_call = lambda: reference(*[ins[n] for n in in_names])  # noqa: E731
        ref = ref_call()
        torch.cuda.synchronize()
        refs = dict(zip(_OUT, ref if isinstance(ref, (tuple, list)) else (ref,)))
        ok, max_abs, max_rel = True, 0.0, 0.0
        for name in _OUT:
            got, want = outs[name], refs[name].to(outs[name].dtype)
            if tuple(got.shape) != tuple(want.shape):
                entry["status"] = "INCORRECT_SHAPE"
                return entry
            a, r = _errors(got, want)
            max_abs, max_rel = max(max_abs, a), max(max_rel, r)
            rtol, atol = cfg.tolerances.get(name, cfg.default_tol)
            ok &= bool(torch.allclose(got.double(), want.double(), rtol=rtol, atol=atol))
        entry["max_abs_error"] = max_abs
        entry["max_rel_error"] = max_rel
        lat = _time_ms(lambda: kernel(*args), cfg.warmup_runs, cfg.iterations, cfg.num_trials)
        ref_lat = _time_ms(ref_call, 1, max(1, cfg.reference_iterations), 1)
        entry["latency_ms"] = lat
        entry["reference_latency_ms"] = ref_lat
        entry["speedup_factor"] = ref_lat / lat if lat > 0 else math.inf
        entry["status"] = "PASSED" if ok else "INCORRECT_NUMERICAL"
    except (ValueError, RuntimeError) as exc:
        entry["error"] = f"{type(exc).__name__}: {exc}"
    return entry


def run_benchmark(trace_set: TraceSet, definitions=None, cfg: BenchmarkConfig | None = None,
                  device=None) -> dict:
    """{definition: {workload uuid: entry}} for the selected definitions (default: every
    definition this library implements that has workloads)."""
    cfg = cfg or BenchmarkConfig()
    if device is None:
        if not torch.cuda.is_available():
            raise RuntimeError("the trace runner needs a ROCm GPU")
        device = torch.device("cuda", torch.cuda.current_device())
    if definitions is None:
        definitions = [n for n in trace_set.definitions
                       if n.startswith(("gdn_decode", "gdn_prefill")) and trace_set.workloads.get(n)]
    results = {}
    for name in definitions:
        if name not in trace_set.definitions:
            raise ValueError(f"Definition '{name}' not found in trace set")
        wls = trace_set.workloads.get(name, [])
        if not wls:
            raise ValueError(f"No workloads found for definition '{name}'")
        defn = trace_set.definitions[name]
        results[name] = {wl.uuid: run_workload(defn, wl, trace_set.root, cfg, device) for wl in wls}
    return results


def print_results(results: dict, file=sys.stdout) -> None:
    """One line per workload, in run_local.py's format (run_local.py:79-101)."""
    for def_name, traces in results.items():
        print(f"\n{def_name}:", file=file)
        for uuid, r in traces.items():
            line = f"  Workload {uuid[:8]}...: {r.get('status')}"
            if r.get("latency_ms") is not None:
                line += f" | {r['latency_ms']:.3f} ms"
            if r.get("speedup_factor") is not None:
                line += f" | {r['speedup_factor']:.2f}x speedup"
            if r.get("max_abs_error") is not None:
                line += f" | abs_err={r['max_abs_error']:.2e}, rel_err={r.get('max_rel_error', 0):.2e}"
            if r.get("error"):
                line += f" | {r['error']}"
            print(line, file=file)


def make_definition(kind: str, hq: int = 16, hk: int = 16, hv: int = 32, d: int = 128) -> dict:
    """A FlashInfer-Trace definition of this path's decode or prefill op with the given
    heads, named like the contest's (``gdn_{decode,prefill}_qk{hq}_v{hv}_d{d}_k_last``,
    config.toml:6,19).  Inputs and outputs follow the reference's DPS parameter order."""
    if kind not in ("decode", "prefill"):
        raise ValueError(f"unknown op {kind!r}")
    axes = {"num_q_heads": {"type": "const", "value": hq},
            "num_k_heads": {"type": "const", "value": hk},
            "num_v_heads": {"type": "const", "value": hv},
            "head_size": {"type": "const", "value": d}}
    sq = lambda *a: {"shape": list(a), "dtype": "bfloat16"}  # noqa: E731
    f32 = lambda *a: {"shape": list(a), "dtype": "float32"}  # noqa: E731
    scalar = {"shape": None, "dtype": "float32"}
    if kind == "decode":
        axes.update(batch_size={"type": "var"}, seq_len={"type": "const", "value": 1})
        lead = ("batch_size", "seq_len")
        inputs = {"q": sq(*lead, "num_q_heads", "head_size"), "k": sq(*lead, "num_k_heads", "head_size"),
                  "v": sq(*lead, "num_v_heads", "head_size"),
                  "state": f32("batch_size", "num_v_heads", "head_size", "head_size"),
                  "A_log": f32("num_v_heads"), "a": sq(*lead, "num_v_heads"),
                  "dt_bias": f32("num_v_heads"), "b": sq(*lead, "num_v_heads"), "scale": scalar}
        outputs = {"output": sq(*lead, "num_v_heads", "head_size"),
                   "new_state": f32("batch_size", "num_v_heads", "head_size", "head_size")}
    else:
        axes.update(total_seq_len={"type": "var"}, num_seqs={"type": "var"},
                    len_cu_seqlens={"type": "var"})
        inputs = {"q": sq("total_seq_len", "num_q_heads", "head_size"),
                  "k": sq("total_seq_len", "num_k_heads", "head_size"),
                  "v": sq("total_seq_len", "num_v_heads", "head_size"),
                  "state": f32("num_seqs", "num_v_heads", "head_size", "head_size"),
                  "A_log": f32("num_v_heads"), "a": sq("total_seq_len", "num_v_heads"),
                  "dt_bias": f32("num_v_heads"), "b": sq("total_seq_len", "num_v_heads"),
                  "cu_seqlens": {"shape": ["len_cu_seqlens"], "dtype": "int32"}, "scale": scalar}
        outputs = {"output": sq("total_seq_len", "num_v_heads", "head_size"),
                   "new_state": f32("num_seqs", "num_v_heads", "head_size", "head_size")}
    return {"name": f"gdn_{kind}_qk{hq}_v{hv}_d{d}_k_last", "op_type": "gdn",
            "description": f"Gated DeltaNet {kind}, k-last fp32 state (this library's layout)",
            "axes": axes, "inputs": inputs, "outputs": outputs}


def write_trace_set(root, definitions, workloads) -> Path:
    """Write a FlashInfer-Trace directory: ``definitions`` are dicts (make_definition);
    ``workloads`` are (definition name, uuid, axes, tensors, scalars) tuples whose
    tensors go to one safetensors blob per workload."""
    from safetensors.torch import save_file
    root = Path(root)
    for d in definitions:
        path = root / "definitions" / d.get("op_type", "misc") / f"{d['name']}.json"
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text(json.dumps(d, indent=2))
    lines = {}
    for name, uuid, axes, tensors, scalars in workloads:
        blob = Path("blob") / "workloads" / f"{name}_{uuid}.safetensors"
        (root / blob).parent.mkdir(parents=True, exist_ok=True)
        save_file({k: v.detach().cpu().contiguous() for k, v in tensors.items()}, str(root / blob))
        inputs = {k: {"type": "safetensors", "path": str(blob), "tensor_key": k} for k in tensors}
        inputs.update({k: {"type": "scalar", "value": v} for k, v in scalars.items()})
        lines.setdefault(name, []).append(json.dumps(
            {"definition": name, "solution": None, "evaluation": None,
             "workload": {"uuid": uuid, "axes": axes, "inputs": inputs}}))
    for name, ls in lines.items():
        path = root / "workloads" / "gdn" / f"{name}.jsonl"
        path.parent.mkdir(parents=True, exist_ok=True)
        path.write_text("\n".join(ls) + "\n")
    return root


def workload_entry(kind: str, uuid: str, inputs: dict):
    """(definition name, uuid, axes, tensors, scalars) for write_trace_set from an input
    dict of ``gdn_kernel_amd.workloads`` (decode_inputs / prefill_inputs)."""
    hq, hk, hv = inputs["q"].shape[-2], inputs["k"].shape[-2], inputs["v"].shape[-2]
    d = inputs["q"].shape[-1]
    name = make_definition(kind, hq, hk, hv, d)["name"]
    names = ["q", "k", "v", "state", "A_log", "a", "dt_bias", "b"]
    if kind == "prefill":
        names.append("cu_seqlens")
    tensors = {n: inputs[n] for n in names}
    if tensors["state"] is None:  # a zero initial state is written out explicitly
        n_state = inputs["q"].shape[0] if kind == "decode" else inputs["cu_seqlens"].numel() - 1
        tensors["state"] = torch.zeros((n_state, hv, inputs["v"].shape[-1], d), dtype=torch.float32)
    if kind == "decode":
        axes = {"batch_size": int(inputs["q"].shape[0])}
    else:
        tensors["cu_seqlens"] = tensors["cu_seqlens"].to(torch.int32)
        axes = {"total_seq_len": int(inputs["q"].shape[0]),
                "num_seqs": int(inputs["cu_seqlens"].numel() - 1),
                "len_cu_seqlens": int(inputs["cu_seqlens"].numel())}
    return name, uuid, axes, tensors, {"scale": float(inputs["scale"])}


def make_dataset(root, configs=(1, 3, 4)) -> Path:
    """A local trace set holding the benchmark configurations of this path
    (``gdn_kernel_amd.workloads.config``) as FlashInfer-Trace workloads."""
    from . import workloads as W
    entries, defs = [], {}
    for c in configs:
        inp = W.config(c)
        kind = "decode" if c in (0, 1, 2) else "prefill"
        if c == 2:
            raise ValueError("config 2 (pooled decode) has no FlashInfer definition")
        e = workload_entry(kind, f"config{c}", inp)
        defs[e[0]] = make_definition(kind)
        entries.append(e)
    return write_trace_set(root, list(defs.values()), entries)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--dataset", default=os.environ.get("FIB_DATASET_PATH"),
                    help="FlashInfer-Trace root (default: $FIB_DATASET_PATH)")
    ap.add_argument("--definition", action="append", help="definition name (repeatable)")
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--iterations", type=int, default=100)
    ap.add_argument("--trials", type=int, default=5)
    ap.add_argument("--reference-iterations", type=int, default=3)
    ap.add_argument("--definition-reference", action="store_true",
                    help="use the definitions' own reference code (executes dataset code)")
    ap.add_argument("--json", help="also write the results to this file")
    ap.add_argument("--make-dataset", metavar="DIR",
                    help="write this path's benchmark configurations 1, 3 and 4 as a "
                         "FlashInfer-Trace set under DIR and exit")
    args = ap.parse_args(argv)
    if args.make_dataset:
        print(f"wrote {make_dataset(args.make_dataset)}")
        return 0
    if not args.dataset:
        print("FIB_DATASET_PATH is not set and no --dataset given", file=sys.stderr)
        return 2
    ts = TraceSet.from_path(args.dataset)
    cfg = BenchmarkConfig(warmup_runs=args.warmup, iterations=args.iterations,
                          num_trials=args.trials, reference_iterations=args.reference_iterations,
                          use_definition_reference=args.definition_reference)
    results = run_benchmark(ts, args.definition, cfg)
    print_results(results)
    if args.json:
        Path(args.json).write_text(json.dumps(results, indent=2))
    bad = [r for t in results.values() for r in t.values() if r.get("status") != "PASSED"]
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main())
