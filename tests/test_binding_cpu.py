"""CPU tests of the Python binding's argument checks and of the workload
generators (no GPU; nothing is launched)."""
import math

import numpy as np
import pytest
import torch

from gdn_kernel_amd import binding, workloads


def test_binding_rejects_cpu_tensors():
    w = workloads.decode_inputs(2, seed=0)
    out = torch.empty_like(w["v"])
    with pytest.raises(ValueError, match="GPU"):
        binding.decode_kernel(w["q"], w["k"], w["v"], w["state"], w["A_log"], w["a"],
                              w["dt_bias"], w["b"], w["scale"], out, w["state"])
    p = workloads.prefill_inputs([3, 5], seed=0)
    with pytest.raises(ValueError, match="GPU"):
        binding.prefill_kernel(p["q"], p["k"], p["v"], p["state"], p["A_log"], p["a"],
                               p["dt_bias"], p["b"], p["cu_seqlens"], p["scale"],
                               torch.empty_like(p["v"]), torch.empty_like(p["state"]))


def test_prefill_with_workspace_checks_arguments():
    p = workloads.prefill_inputs([3, 5], seed=0)
    with pytest.raises(ValueError, match="GPU"):
        binding.prefill_kernel_with_workspace(
            p["q"], p["k"], p["v"], p["state"], p["A_log"], p["a"], p["dt_bias"], p["b"],
            p["cu_seqlens"], p["scale"], torch.empty_like(p["v"]), torch.empty_like(p["state"]),
            torch.empty(16, dtype=torch.uint8))


def test_entry_points_have_reference_arity():
    import inspect
    from gdn_kernel_amd import decode, prefill
    assert list(inspect.signature(decode.kernel).parameters) == [
        "q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "scale", "output", "new_state"]
    assert list(inspect.signature(prefill.kernel).parameters) == [
        "q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens", "scale", "output",
        "new_state"]


def test_decode_inputs_distribution():
    w = workloads.decode_inputs(64, seed=1)
    assert w["q"].dtype == torch.bfloat16 and w["q"].shape == (64, 1, 16, 128)
    n = w["q"].float().norm(dim=-1)
    assert torch.allclose(n, torch.ones_like(n), atol=1e-2)
    A = torch.exp(w["A_log"])
    assert (A >= 1).all() and (A <= 16).all()
    assert w["state"].shape == (64, 32, 128, 128)
    assert abs(float(w["state"].std()) - 0.05) < 1e-3
    assert w["scale"] == 1 / math.sqrt(128)


def test_pool_indices_are_distinct_permutation():
    w = workloads.decode_inputs(512, seed=2, pool_slots=1024)
    idx = w["state_indices"]
    assert idx.dtype == torch.int32 and idx.shape == (512,)
    assert len(set(idx.tolist())) == 512 and int(idx.min()) >= 0 and int(idx.max()) < 1024


def test_varlen_lengths():
    lens = workloads.varlen_lengths(32, 32768)
    assert len(lens) == 32 and sum(lens) == 32768
    assert min(lens) >= 1 and min(lens) < 64 and max(lens) >= 4096 // 2
    assert lens == workloads.varlen_lengths(32, 32768)          # deterministic


def test_prefill_inputs_layout():
    p = workloads.prefill_inputs([5, 0, 70], seed=3, cu_dtype=torch.int64)
    assert p["q"].shape == (75, 16, 128) and p["v"].shape == (75, 32, 128)
    assert p["cu_seqlens"].tolist() == [0, 5, 5, 75] and p["cu_seqlens"].dtype == torch.int64
    assert p["state"].shape == (3, 32, 128, 128)


def test_to_numpy_exact():
    x = torch.randn(100).to(torch.bfloat16)
    y = workloads.to_numpy(x)
    assert y.dtype == np.float64 and np.array_equal(y, x.float().numpy().astype(np.float64))
