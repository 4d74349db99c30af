"""Launches on several streams at once.  The kernels keep nothing between calls (the
prefill hand-offs live in each workgroup's LDS; a workspace belongs to one call; the
library's two scratch arrays are each ordered between launches by an event), so decode
and prefill batches running concurrently on separate streams give the results of the
same calls run one after another, bit for bit."""
import pytest
import torch

from gdn_kernel_amd import _lib, binding, workloads
from tests.gpu_util import say

pytestmark = pytest.mark.gpu


def _outputs(p, N):
    T, Hv = p["v"].shape[0], p["v"].shape[1]
    return (torch.full((T, Hv, 128), float("nan"), device=p["v"].device, dtype=torch.bfloat16),
            torch.full((N, Hv, 128, 128), float("nan"), device=p["v"].device, dtype=torch.float32))


def _no_alloc(p, o, st):
    """gdn_prefill_no_alloc through the C ABI on the current stream."""
    lib = _lib.load()
    T, Hq, Hk, Hv = p["q"].shape[0], p["q"].shape[1], p["k"].shape[1], p["v"].shape[1]
    N = p["cu_seqlens"].numel() - 1
    ptr = lambda t: None if t is None else t.data_ptr()
    _lib.check(lib.gdn_prefill_no_alloc(
        ptr(p["q"]), ptr(p["k"]), ptr(p["v"]), ptr(p["state"]), ptr(p["A_log"]), ptr(p["a"]),
        ptr(p["dt_bias"]), ptr(p["b"]), p["cu_seqlens"].data_ptr(), _lib.GDN_INDEX_INT32, N, T,
        p["scale"], ptr(o), ptr(st), Hq, Hk, Hv, 128, 128, torch.cuda.current_stream().cuda_stream))


def test_concurrent_streams_match_sequential(gpu):
    """Eight streams: decode B=64 out of place; prefill with 128 chains (split 2 ways);
    prefill with 32 chains (split 8 ways); the same 32 chains with a workspace (prep
    kernel + state pass); two drop-in calls on one 3,000-token sequence, which run the
    two-kernel path in the library's drop-in scratch; and two gdn_prefill_no_alloc calls
    on 2,000-token sequences, in the library's other scratch (each array ordered between
    the streams by the library).  Each stream launches its call three times with no
    synchronisation in between."""
    say("concurrent streams: decode B=64, prefill 128 chains, 32 chains, 32 chains with a workspace, "
        "two 3,000-token drop-in calls, two 2,000-token no-alloc calls")
    w = workloads.decode_inputs(64, seed=51, device=gpu, gate="slow", state_scale=0.5)
    pa = workloads.prefill_inputs([700, 64, 5, 300], seed=52, device=gpu, gate="slow", state_scale=0.5)
    pb = workloads.prefill_inputs([900], seed=53, device=gpu, gate="slow", state_scale=0.5)
    pc = workloads.prefill_inputs([3000], seed=54, device=gpu, gate="slow", state_scale=0.5)
    pd = workloads.prefill_inputs([3000], seed=55, device=gpu, gate="slow", state_scale=0.5)
    dec_o, dec_s = torch.empty_like(w["v"]), torch.empty_like(w["state"])
    a_o, a_s = _outputs(pa, 4)
    b_o, b_s = _outputs(pb, 1)
    c_o, c_s = _outputs(pb, 1)
    e_o, e_s = _outputs(pc, 1)
    f_o, f_s = _outputs(pd, 1)
    pg = workloads.prefill_inputs([2000], seed=56, device=gpu, gate="slow", state_scale=0.5)
    ph = workloads.prefill_inputs([2000], seed=57, device=gpu, gate="slow", state_scale=0.5)
    g_o, g_s = _outputs(pg, 1)
    h_o, h_s = _outputs(ph, 1)
    T, Hv = pb["v"].shape[0], pb["v"].shape[1]
    nbytes = binding.prefill_workspace_bytes(1, T, Hv)
    assert nbytes > 0, "the 32-chain batch is expected to take the two-kernel path"
    ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)

    def pre(p, o, s):
        return (p["q"], p["k"], p["v"], p["state"], p["A_log"], p["a"], p["dt_bias"], p["b"],
                p["cu_seqlens"], p["scale"], o, s)

    calls = [
        lambda: binding.decode_kernel(w["q"], w["k"], w["v"], w["state"], w["A_log"], w["a"],
                                      w["dt_bias"], w["b"], w["scale"], dec_o, dec_s),
        lambda: binding.prefill_kernel(*pre(pa, a_o, a_s)),
        lambda: binding.prefill_kernel(*pre(pb, b_o, b_s)),
        lambda: binding.prefill_kernel_with_workspace(*pre(pb, c_o, c_s), ws),
        lambda: binding.prefill_kernel(*pre(pc, e_o, e_s)),
        lambda: binding.prefill_kernel(*pre(pd, f_o, f_s)),
        lambda: _no_alloc(pg, g_o, g_s),
        lambda: _no_alloc(ph, h_o, h_s),
    ]
    results = [(dec_o, dec_s), (a_o, a_s), (b_o, b_s), (c_o, c_s), (e_o, e_s), (f_o, f_s),
               (g_o, g_s), (h_o, h_s)]

    for call in calls:                          # one after another on the current stream
        call()
    torch.cuda.synchronize()
    ref = [(o.clone(), s.clone()) for o, s in results]
    assert torch.equal(ref[2][0], ref[3][0]) and torch.equal(ref[2][1], ref[3][1])
    for o, s in results:
        o.fill_(float("nan"))
        s.fill_(float("nan"))

    streams = [torch.cuda.Stream() for _ in calls]
    main = torch.cuda.current_stream()
    for s in streams:
        s.wait_stream(main)                     # inputs and the NaN fills are ready
    for _ in range(3):
        for s, call in zip(streams, calls):
            with torch.cuda.stream(s):
                call()
    for s in streams:
        main.wait_stream(s)
    torch.cuda.synchronize()
    for i, ((o, s), (ro, rs)) in enumerate(zip(results, ref)):
        assert torch.equal(o, ro), f"stream {i}: output differs from the sequential run"
        assert torch.equal(s, rs), f"stream {i}: state differs from the sequential run"
