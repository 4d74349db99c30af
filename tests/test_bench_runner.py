"""The offline FlashInfer-Trace runner (gdn_kernel_amd.bench_runner): trace-set
round trips, input materialisation, its PyTorch reference against the CPU oracle,
result formatting, and (GPU) an end-to-end evaluation of both definitions."""
import io
import json

import numpy as np
import pytest
import torch

from gdn_kernel_amd import bench_runner as br
from gdn_kernel_amd import reference as R
from gdn_kernel_amd import workloads as W
from gdn_kernel_amd.workloads import Heads, to_numpy
from oracle import gdn_oracle as O
from tests.conftest import assert_close

H = Heads(4, 4, 8)


@pytest.fixture
def small_set(tmp_path):
    p = W.prefill_inputs([70, 5, 0], H, seed=1, gate="slow", state_scale=0.5)
    d = W.decode_inputs(3, H, seed=2, gate="slow", state_scale=0.5)
    root = br.write_trace_set(
        tmp_path, [br.make_definition("prefill", 4, 4, 8), br.make_definition("decode", 4, 4, 8)],
        [br.workload_entry("prefill", "prefill-1", p), br.workload_entry("decode", "decode-1", d)])
    return root, p, d


def test_trace_set_round_trip(small_set):
    root, p, d = small_set
    ts = br.TraceSet.from_path(root)
    assert set(ts.definitions) == {"gdn_prefill_qk4_v8_d128_k_last", "gdn_decode_qk4_v8_d128_k_last"}
    defn = ts.definitions["gdn_prefill_qk4_v8_d128_k_last"]
    (wl,) = ts.workloads[defn.name]
    assert wl.uuid == "prefill-1"
    axes = br.resolve_axes(defn, wl)
    assert axes["total_seq_len"] == 75 and axes["num_seqs"] == 3 and axes["num_v_heads"] == 8
    ins = br.materialize_inputs(defn, wl, root, "cpu")
    assert list(ins) == list(defn.inputs)             # call order kept
    for name in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens"):
        assert torch.equal(ins[name], p[name].to(ins[name].dtype)), name
    assert ins["scale"] == pytest.approx(p["scale"])
    outs = br.allocate_outputs(defn, axes, "cpu")
    assert outs["output"].shape == (75, 8, 128) and outs["output"].dtype == torch.bfloat16
    assert outs["new_state"].shape == (3, 8, 128, 128) and torch.isnan(outs["new_state"]).all()


def test_workload_errors(small_set):
    root, _, _ = small_set
    ts = br.TraceSet.from_path(root)
    defn = ts.definitions["gdn_decode_qk4_v8_d128_k_last"]
    with pytest.raises(ValueError, match="no value for axis 'batch_size'"):
        br.resolve_axes(defn, br.Workload(defn.name, "x", {}, {}))
    with pytest.raises(ValueError, match="unknown axes"):
        br.resolve_axes(defn, br.Workload(defn.name, "x", {"batch_size": 2, "bogus": 1}, {}))
    # random inputs: deterministic per (uuid, name), floats only
    wl = br.Workload(defn.name, "r1", {"batch_size": 2}, {"scale": {"type": "scalar", "value": 0.5}})
    a1 = br.materialize_inputs(defn, wl, root, "cpu")
    a2 = br.materialize_inputs(defn, wl, root, "cpu")
    assert all(torch.equal(a1[n], a2[n]) for n in a1 if torch.is_tensor(a1[n]))
    assert a1["q"].shape == (2, 1, 4, 128) and a1["scale"] == 0.5
    pdef = ts.definitions["gdn_prefill_qk4_v8_d128_k_last"]
    wl = br.Workload(pdef.name, "r2", {"total_seq_len": 4, "num_seqs": 1, "len_cu_seqlens": 2}, {})
    with pytest.raises(ValueError, match="random integer"):
        br.materialize_inputs(pdef, wl, root, "cpu")
    with pytest.raises(ValueError, match="not found"):
        br.run_benchmark(ts, ["gdn_nope"], device=torch.device("cpu"))


def test_unsupported_definition_is_reported():
    defn = br.Definition.from_json({"name": "moe_x", "axes": {}, "inputs": {}, "outputs": {}})
    r = br.run_workload(defn, br.Workload("moe_x", "u", {}, {}), ".", br.BenchmarkConfig(), "cpu")
    assert r["status"] == "UNSUPPORTED_DEFINITION"


def test_definition_reference_is_loaded_from_its_source():
    src = "def run(x, y):\n    return x + y\n"
    defn = br.Definition.from_json({"name": "gdn_decode_t", "axes": {}, "inputs": {},
                                    "outputs": {}, "reference": src})
    assert br._definition_reference(defn)(2, 3) == 5
    with pytest.raises(ValueError, match="no run"):
        br._definition_reference(br.Definition.from_json(
            {"name": "d", "axes": {}, "inputs": {}, "outputs": {}, "reference": "x = 1\n"}))


def test_print_results_format():
    buf = io.StringIO()
    br.print_results({"gdn_decode_x": {"0123456789ab": {
        "status": "PASSED", "solution": br.SOLUTION_NAME, "latency_ms": 0.0123,
        "reference_latency_ms": 0.5, "speedup_factor": 40.65, "max_abs_error": 1e-3,
        "max_rel_error": 2e-3}}}, file=buf)
    assert ("Workload 01234567...: PASSED | 0.012 ms | 40.65x speedup | "
            "abs_err=1.00e-03, rel_err=2.00e-03") in buf.getvalue()


def test_main_without_dataset(monkeypatch, capsys):
    monkeypatch.delenv("FIB_DATASET_PATH", raising=False)
    assert br.main([]) == 2


@pytest.mark.parametrize("gate", ["baseline", "slow"])
def test_torch_decode_reference_matches_oracle(gate):
    d = W.decode_inputs(3, H, seed=5, gate=gate, state_scale=0.5)
    o, s = R.decode_reference(d["q"], d["k"], d["v"], d["state"], d["A_log"], d["a"],
                              d["dt_bias"], d["b"], d["scale"])
    o_ref, s_ref = O.decode(*[to_numpy(d[n]) for n in ("q", "k", "v", "state", "A_log", "a",
                                                       "dt_bias", "b")], d["scale"])
    assert_close(to_numpy(o), o_ref, 1e-2, 1e-2, "output")
    assert_close(to_numpy(s), s_ref, 1e-4, 1e-6, "state")


@pytest.mark.parametrize("gate", ["baseline", "slow"])
def test_torch_prefill_reference_matches_sequential_definition(gate):
    p = W.prefill_inputs([130, 7, 0, 64], H, seed=6, gate=gate, state_scale=0.5)
    o, s = R.prefill_reference(p["q"], p["k"], p["v"], p["state"], p["A_log"], p["a"],
                               p["dt_bias"], p["b"], p["cu_seqlens"], p["scale"])
    o_ref, s_ref = O.prefill_sequential(*[to_numpy(p[n]) for n in ("q", "k", "v", "state", "A_log",
                                                                   "a", "dt_bias", "b")],
                                        p["cu_seqlens"].numpy(), p["scale"])
    assert_close(to_numpy(o), o_ref, 1e-2, 1e-2, "output")
    assert_close(to_numpy(s), s_ref, 1e-4, 1e-6, "state")
    assert torch.equal(s[2], p["state"][2])          # empty sequence passes its state through


@pytest.mark.gpu
@pytest.mark.parametrize("definition_reference", [False, True])
def test_runner_end_to_end(gpu, small_set, definition_reference):
    root, _, _ = small_set
    ts = br.TraceSet.from_path(root)
    if definition_reference:
        # The definitions' own reference code, as the harness would run it.
        for name, defn in ts.definitions.items():
            fn = "decode_reference" if "decode" in name else "prefill_reference"
            defn.reference = (f"from gdn_kernel_amd.reference import {fn}\n"
                              f"def run(**kw):\n    return {fn}(**kw)\n")
    cfg = br.BenchmarkConfig(warmup_runs=1, iterations=5, num_trials=2, reference_iterations=1,
                             use_definition_reference=definition_reference)
    res = br.run_benchmark(ts, None, cfg, gpu)
    assert set(res) == set(ts.definitions)
    for name, entries in res.items():
        for uuid, r in entries.items():
            assert r["status"] == "PASSED", (name, uuid, r)
            assert r["latency_ms"] > 0 and r["reference_latency_ms"] > 0 and r["speedup_factor"] > 0
            assert r["max_abs_error"] < 1e-1
    json.dumps(res)                                   # serialisable as the harness's results


def test_tools_cli_errors(small_set, monkeypatch):
    from gdn_kernel_amd import tools
    root, _, _ = small_set
    monkeypatch.delenv("FIB_DATASET_PATH", raising=False)
    assert tools.main(["sanitize", "--definition", "x"]) == 2
    with pytest.raises(ValueError, match="unknown sanitizer"):
        tools.run_sanitizer(root, "gdn_decode_qk4_v8_d128_k_last", sanitizer_types=("bogus",))
    with pytest.raises(ValueError, match="no workload"):
        tools._pick(br.TraceSet.from_path(root), "gdn_decode_qk4_v8_d128_k_last", "nope")


def test_guard_regions_detect_writes():
    from gdn_kernel_amd import tools
    t = torch.arange(10, dtype=torch.float32)
    inner, back = tools._guarded_like(t)
    assert torch.equal(inner, t) and inner.data_ptr() - back.data_ptr() == tools.GUARD_BYTES
    assert tools._guards_intact(back, 40)
    back[tools.GUARD_BYTES + 40] = 0                  # one byte past the end
    assert not tools._guards_intact(back, 40)


@pytest.mark.gpu
def test_sanitizer_checks_pass(gpu, small_set):
    from gdn_kernel_amd import tools
    root, _, _ = small_set
    for name in ("gdn_decode_qk4_v8_d128_k_last", "gdn_prefill_qk4_v8_d128_k_last"):
        rep = tools.run_sanitizer(root, name, sanitizer_types=("initcheck", "memcheck", "racecheck"),
                                  device=gpu)
        assert rep.endswith("SANITIZER SUMMARY: 0 error(s)"), rep
        assert "initcheck: PASSED" in rep and "memcheck: PASSED" in rep and "racecheck: PASSED" in rep


@pytest.mark.gpu
def test_profiler_wrapper_kernel_trace(gpu, small_set, tmp_path):
    from gdn_kernel_amd import tools
    root, _, _ = small_set
    rep = tools.run_profiler(root, "gdn_decode_qk4_v8_d128_k_last", iterations=5,
                             out_dir=tmp_path / "prof", timeout=240)
    assert "gdn_decode_kernel" in rep, rep
    row = [ln for ln in rep.splitlines() if "gdn_decode_kernel" in ln][0]
    assert int(row.split()[-4]) == 5                  # calls
