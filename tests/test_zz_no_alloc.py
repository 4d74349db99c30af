"""gdn_prefill_no_alloc: the prefill entry point that allocates nothing (its chunk
images live in the library's per-device scratch array) against
gdn_prefill_with_workspace (the same kernels with a caller-owned workspace), through
the C ABI, on two calls in a row -- a batch that fills most of the scratch, then a
smaller one -- and the rejection of a batch whose images exceed the scratch."""
import ctypes

import pytest
import torch

from gdn_kernel_amd import _lib, workloads
from gdn_kernel_amd.workloads import Heads
from tests.gpu_util import say

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = _lib.GDN_PREFILL_NO_ALLOC_SCRATCH_BYTES  # 64 MiB, as in the header


def _call(lib, fn, p, gpu, ws=None):
    d = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in p.items()}
    T, Hq = d["q"].shape[0], d["q"].shape[1]
    Hk, Hv = d["k"].shape[1], d["v"].shape[1]
    cu = d["cu_seqlens"]
    N = cu.numel() - 1
    out = torch.full((T, Hv, 128), float("nan"), device=gpu, dtype=torch.bfloat16)
    ns = torch.full((N, Hv, 128, 128), float("nan"), device=gpu, dtype=torch.float32)
    ptr = lambda t: None if t is None else t.data_ptr()
    args = [ptr(d["q"]), ptr(d["k"]), ptr(d["v"]), ptr(d["state"]), ptr(d["A_log"]), ptr(d["a"]),
            ptr(d["dt_bias"]), ptr(d["b"]), cu.data_ptr(), _lib.GDN_INDEX_INT32, N, T, d["scale"],
            ptr(out), ptr(ns), Hq, Hk, Hv, 128, 128]
    stream = torch.cuda.current_stream(gpu).cuda_stream
    if fn == "with_workspace":
        rc = lib.gdn_prefill_with_workspace(*args, ws.data_ptr(), ws.numel(), stream)
    else:
        rc = lib.gdn_prefill_no_alloc(*args, stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return out, ns


def test_prefill_no_alloc_matches_workspace_entry_point(gpu):
    lib = _lib.load()
    big = workloads.prefill_inputs([4096], seed=51, gate="slow", state_scale=0.5)     # config 3 shape
    small = workloads.prefill_inputs([150, 64, 7, 0], Heads(4, 4, 8), seed=52, gate="slow",
                                     state_scale=0.5)
    for name, p in (("large", big), ("smaller", small)):
        T, Hv, N = p["q"].shape[0], p["v"].shape[1], len(p["lengths"])
        need = lib.gdn_prefill_workspace_size(N, T, Hv)
        assert 0 < need <= SCRATCH_BYTES, need
        say(f"prefill no-alloc vs workspace: {name} batch, {need} bytes of chunk images")
        ws = torch.full((need,), 0xA5, device=gpu, dtype=torch.uint8)
        o_ref, s_ref = _call(lib, "with_workspace", p, gpu, ws)
        o, s = _call(lib, "no_alloc", p, gpu)
        assert torch.equal(o, o_ref) and torch.equal(s, s_ref), f"{name}: results differ"


def test_prefill_no_alloc_rejects_batches_beyond_its_scratch(gpu):
    lib = _lib.load()
    p = workloads.prefill_inputs([4096, 4096], seed=53)     # 64 chains: 78.6 MB of chunk images
    need = lib.gdn_prefill_workspace_size(2, 8192, 32)
    assert need > SCRATCH_BYTES
    say("prefill no-alloc: batch beyond the scratch is rejected")
    with pytest.raises(ValueError, match="scratch"):
        _call(lib, "no_alloc", p, gpu)
