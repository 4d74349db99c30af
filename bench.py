#!/usr/bin/env python3
"""Benchmark of the MI355X GDN hot path; prints ONE JSON line.

Headline (``value``): GDN decode at B=64 (heads 16/16/32, dk=dv=128, fp32 state
[64,32,128,128] updated in place) as algorithmic HBM GB/s:
  bytes/step = 2*B*Hv*dv*dk*4 (state in + out) + B*(2*Hq*dk*2 + 2*Hv*dv*2 + 2*Hv*2)
               (q, k, v, output, a, b) + 2*Hv*4 (A_log, dt_bias) = 270,016,768 B.
Inputs are resident in HBM before the timed region.  To keep the 256 MB
Infinity Cache from serving the state, steps rotate over 4 independent state
buffers (537 MB).

Also reported on the same line: pooled decode (B=512 over a 1024-slot pool),
chunked prefill tokens/s on the 32-sequence / 32768-token varlen batch and on
the single 4096-token sequence (with MFMA-roofline fractions computed from the
algorithmic 180,224 FLOP per token and v-head), the rates this box measures on
library work (a device copy and a bf16 GEMM, ``measured_peaks``) with the roofline
fractions against them, and the CPU baseline (the reference's PyTorch decode definition
restated, fp32 on every host core this process may use; the numpy oracle on one thread
is reported beside it).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only decode|prefill]
       [--no-cpu] [--cpu-seconds S]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_BF16_PEAK_TFS = 2516.6    # MI355X dense bf16 MFMA, TFLOP/s
PREFILL_FLOP_PER_TOKEN_HEAD = 180224   # 2*(5*C*d + 3*dk*dv), C=64, d=128
HQ, HK, HV, D = 16, 16, 32, 128


def decode_bytes(B, slots_idx=False):
    b = 2 * B * HV * D * D * 4 + B * (2 * HQ * D * 2 + 2 * HV * D * 2 + 2 * HV * 2) + 2 * HV * 4
    if slots_idx:
        b += 4 * B
    return b


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=["decode", "prefill", "all"], default="all")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--pmc-run", action="store_true",
                    help="short fixed launch sequence for rocprofv3 --pmc runs: a torch copy of "
                         "COPY_BYTES (counter calibration), then 5 decode B=64 launches, 2 "
                         "prefill launches of the 32k varlen batch and 2 of the T=4096 "
                         "sequence (drop-in kernel); prints nothing")
    return ap.parse_args()


PREFILL_WARM_S = 0.3   # untimed prefill launches before timing (clock ramp-up)
PREFILL_CPU_TOKENS = 1024  # CPU prefill baseline sample (tokens of config 4's sequence 0)
COPY_BYTES = 1 << 28   # 256 MiB read + 256 MiB written by the calibration copy


def pmc_run(torch, binding, workloads):
    dev = torch.device("cuda:0")
    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    flush = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev)
    for _ in range(3):
        flush.fill_(1.0)
        dst.copy_(src)
    torch.cuda.synchronize()
    w = workloads.decode_inputs(64, seed=1, device=dev)
    states = [w["state"]] + [w["state"].clone() for _ in range(3)]
    out = torch.empty_like(w["v"])
    for i in range(5):
        flush.fill_(1.0)
        st = states[i % 4]
        binding.decode_kernel(w["q"], w["k"], w["v"], st, w["A_log"], w["a"], w["dt_bias"],
                              w["b"], w["scale"], out, st)
    torch.cuda.synchronize()
    p = workloads.config(4, device=dev)
    po = torch.empty((p["q"].shape[0], HV, D), dtype=torch.bfloat16, device=dev)
    ns = torch.empty_like(p["state"])
    for _ in range(2):
        flush.fill_(1.0)
        binding.prefill_kernel(p["q"], p["k"], p["v"], p["state"], p["A_log"], p["a"],
                               p["dt_bias"], p["b"], p["cu_seqlens"], p["scale"], po, ns)
    torch.cuda.synchronize()
    p = workloads.config(3, device=dev)
    po = torch.empty((p["q"].shape[0], HV, D), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((1, HV, D, D), dtype=torch.float32, device=dev)
    for _ in range(2):
        flush.fill_(1.0)
        binding.prefill_kernel(p["q"], p["k"], p["v"], p["state"], p["A_log"], p["a"],
                               p["dt_bias"], p["b"], p["cu_seqlens"], p["scale"], po, ns)
    torch.cuda.synchronize()


GEMM_N = 8192   # measured bf16 GEMM peak: torch.matmul of two 8192 x 8192 bf16 matrices


def measured_peaks(torch):
    """What this GPU reaches on plain library work, for roofline fractions against
    measured rather than datasheet peaks: a device-to-device copy of COPY_BYTES
    (read + written bytes over time, 4 rotating buffer pairs so the Infinity Cache
    does not serve it) and a bf16 GEMM through torch.matmul (hipBLASLt), both timed
    with HIP events after untimed warm-up."""
    dev = torch.device("cuda:0")
    pairs = [(torch.ones(COPY_BYTES // 4, dtype=torch.float32, device=dev),
              torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev)) for _ in range(4)]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for src, dst in pairs * 2:
        dst.copy_(src)
    torch.cuda.synchronize()
    reps = 20
    e0.record()
    for i in range(reps):
        src, dst = pairs[i % 4]
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    copy_gbs = 2 * COPY_BYTES * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del pairs
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn((GEMM_N, GEMM_N), generator=g, dtype=torch.bfloat16, device=dev)
    b = torch.randn((GEMM_N, GEMM_N), generator=g, dtype=torch.bfloat16, device=dev)
    c = torch.empty((GEMM_N, GEMM_N), dtype=torch.bfloat16, device=dev)
    t_end = time.perf_counter() + 0.3
    while time.perf_counter() < t_end:
        torch.matmul(a, b, out=c)
        torch.cuda.synchronize()
    reps = 20
    e0.record()
    for _ in range(reps):
        torch.matmul(a, b, out=c)
    e1.record()
    torch.cuda.synchronize()
    gemm_tfs = 2 * GEMM_N ** 3 * reps / (e0.elapsed_time(e1) * 1e-3) / 1e12
    return {"copy_gbs": round(copy_gbs, 1), "copy_bytes": 2 * COPY_BYTES,
            "bf16_gemm_tflops": round(gemm_tfs, 1), "gemm_shape": [GEMM_N, GEMM_N, GEMM_N]}


def timed_launches(fn, steps, warmup, torch, use_graph=False):
    """Warm up, then time exactly ``steps`` launches of ``fn(i)``.

    With ``use_graph`` the ``steps`` launches are captured once into a HIP graph
    (torch.cuda.CUDAGraph on the current device), replayed once untimed, and the
    timed region is one replay; otherwise they are launched eagerly.  Returns
    (wall seconds between two synchronisations, mean ms per launch from a HIP
    event pair recorded on the launch stream around the timed region, mode)."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    graph, mode = None, "eager"
    if use_graph:
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                fn(0)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(steps):
                    fn(warmup + i)
            graph.replay()
            torch.cuda.synchronize()
            mode = "hipGraph"
        except Exception as exc:          # capture unsupported: fall back to eager launches
            print(f"bench.py: graph capture failed ({exc}); timing eager launches",
                  file=sys.stderr)
            graph = None
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    if graph is not None:
        graph.replay()
    else:
        for i in range(steps):
            fn(warmup + i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(end) / steps, mode


def bench_decode(args, torch, binding, workloads):
    dev = torch.device("cuda:0")
    B = 64
    nbuf = 4
    w = workloads.decode_inputs(B, seed=1, device=dev)
    states = [w["state"]] + [w["state"].clone() for _ in range(nbuf - 1)]
    out = torch.empty_like(w["v"])

    def step(i):
        st = states[i % nbuf]
        binding.decode_kernel(w["q"], w["k"], w["v"], st, w["A_log"], w["a"], w["dt_bias"],
                              w["b"], w["scale"], out, st)

    wall, ev_ms, mode = timed_launches(step, args.steps, args.warmup, torch, use_graph=True)
    wall_e, ev_ms_e, _ = timed_launches(step, args.steps, 0, torch, use_graph=False)
    return dict(bytes=decode_bytes(B), wall=wall, ev_ms=ev_ms, mode=mode, eager_wall=wall_e,
                eager_ev_ms=ev_ms_e)


DECODE_B1_BUFFERS = 192   # 192 x 2 MiB B=1 states (403 MB) rotate past the 256 MB Infinity Cache


def bench_decode_b1(args, torch, binding, workloads):
    """Single-sequence decode latency on BASELINE config 0's shape (B=1, heads 16/16/32,
    fp32 state updated in place), graph-replayed: "cold" rotates over DECODE_B1_BUFFERS
    independent states so each launch reads its state from HBM; "warm" reuses one state,
    which then stays in the caches."""
    dev = torch.device("cuda:0")
    w = workloads.decode_inputs(1, seed=0, device=dev)
    states = [w["state"]] + [w["state"].clone() for _ in range(DECODE_B1_BUFFERS - 1)]
    out = torch.empty_like(w["v"])

    def run(st):
        binding.decode_kernel(w["q"], w["k"], w["v"], st, w["A_log"], w["a"], w["dt_bias"],
                              w["b"], w["scale"], out, st)

    steps = max(args.steps, 50)
    _, cold_ms, mode = timed_launches(lambda i: run(states[i % DECODE_B1_BUFFERS]), steps,
                                      args.warmup, torch, use_graph=True)
    _, warm_ms, _ = timed_launches(lambda i: run(states[0]), steps, args.warmup, torch,
                                   use_graph=True)
    return {"us": round(cold_ms * 1e3, 3), "us_warm": round(warm_ms * 1e3, 3), "launch": mode,
            "bytes": decode_bytes(1),
            "gbs": round(decode_bytes(1) / (cold_ms * 1e-3) / 1e9, 1),
            "state_buffers": DECODE_B1_BUFFERS}


def bench_pooled(args, torch, binding, workloads):
    dev = torch.device("cuda:0")
    w = workloads.decode_inputs(512, seed=2, device=dev, pool_slots=1024)
    out = torch.empty_like(w["v"])

    def step(i):
        binding.decode_pooled_kernel(w["q"], w["k"], w["v"], w["state"], w["A_log"], w["a"],
                                     w["dt_bias"], w["b"], w["scale"], out, w["state_indices"])

    steps = max(5, args.steps // 2)
    wall, ev_mean, _ = timed_launches(step, steps, min(args.warmup, 3), torch)
    nbytes = decode_bytes(512, slots_idx=True)
    return dict(us=ev_mean * 1e3, gbs=nbytes / (ev_mean * 1e-3) / 1e9,
                frac=nbytes / (ev_mean * 1e-3) / 1e9 / HBM_PEAK_GBS, bytes=nbytes)


# Independent input/output/state sets that cold prefill timing rotates over, so that
# the 256 MB Infinity Cache cannot serve a launch its inputs: config 4 (942 MB a set)
# and config 3 (103 MB a set, plus the drop-in's 58 MB of chunk images, which every
# launch rewrites before it reads them).
PREFILL_COLD_SETS = {4: 3, 3: 4}


def bench_prefill(args, torch, binding, workloads, cfg, path="drop-in", cold=False):
    """Prefill on config ``cfg`` through ``path``: "drop-in" (the reference-signature
    ``kernel``, gdn_prefill), "workspace" (gdn_prefill_with_workspace with a
    preallocated workspace) or "no-alloc" (gdn_prefill_no_alloc, the library's
    scratch).  Warm (default): every launch reuses one input/output/state set.  Cold
    (drop-in only): launches rotate over PREFILL_COLD_SETS[cfg] sets with distinct
    seeds."""
    dev = torch.device("cuda:0")
    nsets = PREFILL_COLD_SETS[cfg] if cold else 1
    sets = []
    for j in range(nsets):
        p = workloads.config(cfg, device=dev, seed=cfg + 100 * j)
        T = p["q"].shape[0]
        N = p["cu_seqlens"].numel() - 1
        out = torch.empty((T, HV, D), dtype=torch.bfloat16, device=dev)
        ns = torch.empty((N, HV, D, D), dtype=torch.float32, device=dev)
        sets.append((p["q"], p["k"], p["v"], p["state"], p["A_log"], p["a"], p["dt_bias"], p["b"],
                     p["cu_seqlens"], p["scale"], out, ns))
    args_ = sets[0]
    if path == "drop-in":
        def step(i):
            binding.prefill_kernel(*sets[i % nsets])
    elif path == "workspace":
        ws = torch.empty(binding.prefill_workspace_bytes(N, T, HV), dtype=torch.uint8, device=dev)

        def step(i):
            binding.prefill_kernel_with_workspace(*args_, ws)
    else:
        from gdn_kernel_amd import _lib
        out, ns = args_[10], args_[11]
        lib = _lib.load()
        ptr = lambda t: None if t is None else t.data_ptr()
        cargs = [ptr(p[k]) for k in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")]
        cargs += [p["cu_seqlens"].data_ptr(), _lib.GDN_INDEX_INT32, N, T, p["scale"], ptr(out),
                  ptr(ns), HQ, HK, HV, D, D]
        stream = torch.cuda.current_stream(dev).cuda_stream

        def step(i):
            _lib.check(lib.gdn_prefill_no_alloc(*cargs, stream))

    # Untimed warm-up for at least PREFILL_WARM_S (the GPU leaves its idle clocks
    # within the first few hundred milliseconds), then `steps` timed launches.
    steps = max(10, args.steps // 2)
    t_end = time.perf_counter() + PREFILL_WARM_S
    nwarm = 0
    while nwarm < max(args.warmup, 2) or time.perf_counter() < t_end:
        step(nwarm)
        nwarm += 1
        if nwarm % 8 == 0:
            torch.cuda.synchronize()
    wall, ev_mean, _ = timed_launches(step, steps, 0, torch)
    flop = HV * T * PREFILL_FLOP_PER_TOKEN_HEAD
    tfs = flop / (ev_mean * 1e-3) / 1e12
    r = dict(tokens=T, seqs=N, us=ev_mean * 1e3, tokens_per_s=T / (ev_mean * 1e-3),
             tflops=tfs, mfma_frac=tfs / MFMA_BF16_PEAK_TFS, flop=flop,
             lengths=p["lengths"] if cfg == 4 else None)
    if cold:
        r["input_sets"] = nsets
    return r


def cpu_model():
    """The host CPU's model name as /proc/cpuinfo reports it for the first processor
    (with its family and model numbers), else platform's description."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break
                key, _, val = line.partition(":")
                info.setdefault(key.strip(), val.strip())
    except OSError:
        pass
    name = info.get("model name") or platform.processor() or platform.machine()
    if "cpu family" in info:
        return f"{name} (family {info['cpu family']}, model {info.get('model', '?')})"
    return name


def cpu_baseline(seconds, workloads, torch):
    """BASELINE config 0 (B=1, heads 16/16/32) through the reference's PyTorch decode
    definition (design.md:166-226, restated in oracle/torch_definition.py), fp32 on the
    host CPU with torch's thread pool on every core this process may run on
    (len(os.sched_getaffinity(0))): one warm-up run, then the median of at least 5 runs
    over about ``seconds``."""
    from oracle.torch_definition import decode_definition
    cores = len(os.sched_getaffinity(0))
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        w = workloads.config(0)
        args = [w[k] for k in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "scale")]
        decode_definition(*args)
        times = []
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end or len(times) < 5:
            t0 = time.perf_counter()
            decode_definition(*args)
            times.append(time.perf_counter() - t0)
    finally:
        torch.set_num_threads(prev)
    med = float(np.median(times))
    nbytes = decode_bytes(1)
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": cores, "kind": "port",
            "us_per_step": med * 1e6,
            "sample": (f"reference PyTorch decode definition (design.md:166-226), fp32, "
                       f"torch.set_num_threads({cores}), on config 0: B=1, 32 v-heads, "
                       f"{nbytes} algorithmic bytes/step; median of {len(times)} steps after "
                       f"1 warm-up, over ~{seconds:.0f} s"),
            "cpu_model": cpu_model()}


def cpu_baseline_numpy(seconds, workloads):
    """The oracle's decode (design.md:166-226 restated in numpy, fp32 arithmetic like the
    reference's .float() path) on BASELINE config 0 (B=1), single-threaded."""
    from threadpoolctl import threadpool_limits
    from oracle import gdn_oracle as O
    w = workloads.config(0)
    a = [workloads.to_numpy(w[k]).astype(np.float32) for k in
         ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")]
    times = []
    with threadpool_limits(limits=1):
        O.decode(*a, w["scale"], dtype=np.float32)
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end or len(times) < 5:
            t0 = time.perf_counter()
            O.decode(*a, w["scale"], dtype=np.float32)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    nbytes = decode_bytes(1)
    return {"value": nbytes / med / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "us_per_step": med * 1e6,
            "sample": (f"oracle decode (numpy fp32, 1 thread) on config 0: B=1, 32 v-heads, "
                       f"{nbytes} algorithmic bytes/step; median of {len(times)} steps over "
                       f"~{seconds:.0f} s")}


def cpu_baseline_prefill(seconds, workloads):
    """The oracle's chunked prefill (kernel_prefill.cu:95-294 restated in numpy, fp32) on a
    bounded sample of config 4: the first PREFILL_CPU_TOKENS tokens of its sequence 0, all
    32 v-heads, from that sequence's initial state; single-threaded."""
    from threadpoolctl import threadpool_limits
    from oracle import gdn_oracle as O
    p = workloads.config(4)
    n = PREFILL_CPU_TOKENS
    assert p["lengths"][0] >= n
    f32 = lambda t: workloads.to_numpy(t).astype(np.float32)
    args = [f32(p["q"][:n]), f32(p["k"][:n]), f32(p["v"][:n]), f32(p["state"][:1]), f32(p["A_log"]),
            f32(p["a"][:n]), f32(p["dt_bias"]), f32(p["b"][:n])]
    cu = np.array([0, n], np.int64)
    times = []
    with threadpool_limits(limits=1):
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            O.prefill_chunked(*args, cu, p["scale"], dtype=np.float32)
            times.append(time.perf_counter() - t0)
    med = float(np.median(times))
    return {"value": n / med, "unit": "tokens/s", "cores": 1, "kind": "port",
            "us_per_sample": med * 1e6,
            "sample": (f"oracle chunked prefill (numpy fp32, 1 thread) on the first {n} tokens "
                       f"of config 4's sequence 0, 32 v-heads, its initial state; median of "
                       f"{len(times)} runs over ~{seconds:.0f} s")}


def load_traffic():
    """HBM bytes per decode launch measured with rocprofv3 PMC counters, if a
    measurement has been recorded under profiles/."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "decode_b64_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes")
    except (OSError, ValueError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the decode and prefill paths shard with no exchange and are measured on one "
              "GPU's share", file=sys.stderr)
        sys.exit(2)
    import torch
    from gdn_kernel_amd import binding, workloads, _lib
    _lib.load()
    assert torch.cuda.is_available(), "no ROCm GPU visible"
    if args.pmc_run:
        pmc_run(torch, binding, workloads)
        return

    res = {"metric": "GDN decode µs + HBM GB/s at B=64; prefill tokens/s (32k varlen), 1 GPU",
           "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": None, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
           "config": {"workload": "GDN decode, B=64, one token, Hq=Hk=16, Hv=32, dk=dv=128, "
                                  "bf16 q/k/v/a/b, fp32 state [64,32,128,128] updated in place "
                                  "(4 rotating state buffers, cold Infinity Cache)",
                      "batch": 64, "heads": [HQ, HK, HV], "head_dim": D}}
    if args.only in ("decode", "all"):
        d = bench_decode(args, torch, binding, workloads)
        gbs_wall = d["bytes"] * args.steps / d["wall"] / 1e9
        gbs_kernel = d["bytes"] / (d["ev_ms"] * 1e-3) / 1e9
        res["value"] = round(gbs_wall, 1)
        res["ms_per_step"] = round(d["wall"] / args.steps * 1e3, 5)
        res["decode_us"] = round(d["ev_ms"] * 1e3, 2)
        res["launch"] = d["mode"]
        res["decode_eager"] = {"us_per_launch": round(d["eager_ev_ms"] * 1e3, 2),
                               "wall_gbs": round(d["bytes"] * args.steps / d["eager_wall"] / 1e9, 1)}
        res["roofline"] = {"bound": "hbm", "achieved": round(gbs_kernel, 1),
                           "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(gbs_kernel / HBM_PEAK_GBS, 4),
                           "traffic": load_traffic(),
                           "kernel": "gdn_decode_kernel", "bytes_per_launch": d["bytes"]}
        pooled = bench_pooled(args, torch, binding, workloads)
        res["decode_pooled_b512"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                     for k, v in pooled.items()}
        res["decode_b1"] = bench_decode_b1(args, torch, binding, workloads)
        res["decode_b1_us"] = res["decode_b1"]["us"]
    if args.only in ("prefill", "all"):
        for cfg, key, path, cold in ((4, "prefill_varlen_32k", "drop-in", False),
                                     (4, "prefill_varlen_32k_cold", "drop-in", True),
                                     (3, "prefill_t4096", "drop-in", False),
                                     (3, "prefill_t4096_cold", "drop-in", True),
                                     (3, "prefill_t4096_workspace", "workspace", False),
                                     (3, "prefill_t4096_no_alloc", "no-alloc", False)):
            pr = bench_prefill(args, torch, binding, workloads, cfg, path, cold)
            pr["path"] = {"drop-in": "kernel (gdn_prefill, as the TVM-FFI shim)",
                          "workspace": "kernel_with_workspace (gdn_prefill_with_workspace)",
                          "no-alloc": "gdn_prefill_no_alloc (library scratch)"}[path]
            res[key] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in pr.items()}
        if res["value"] is None:
            res["value"] = round(res["prefill_varlen_32k"]["tokens_per_s"], 1)
            res["unit"] = "tokens/s"
            res["ms_per_step"] = round(res["prefill_varlen_32k"]["us"] / 1e3, 5)
    # Roofline fractions against what this box measures on library work, beside the
    # datasheet fractions above.
    peaks = measured_peaks(torch)
    res["measured_peaks"] = peaks
    if "roofline" in res:
        res["roofline"]["frac_of_measured_copy"] = round(res["roofline"]["achieved"] / peaks["copy_gbs"], 4)
    for key in ("prefill_varlen_32k", "prefill_varlen_32k_cold", "prefill_t4096",
                "prefill_t4096_cold", "prefill_t4096_workspace", "prefill_t4096_no_alloc"):
        if key in res:
            res[key]["frac_of_measured_gemm"] = round(res[key]["tflops"] / peaks["bf16_gemm_tflops"], 4)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline(args.cpu_seconds, workloads, torch)
        res["cpu_baseline_numpy_1t"] = cpu_baseline_numpy(args.cpu_seconds / 2, workloads)
        if args.only in ("prefill", "all"):
            res["cpu_baseline_prefill"] = cpu_baseline_prefill(args.cpu_seconds / 2, workloads)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
