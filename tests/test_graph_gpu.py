"""HIP-graph capture of the decode and prefill launches: every replay (with eager
work and synchronisations in between) must reproduce the eager result bit for bit."""
import pytest
import torch

from gdn_kernel_amd import _lib, binding, workloads
from tests.gpu_util import say

pytestmark = pytest.mark.gpu


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def test_decode_graph_replays_match_eager(gpu):
    say("decode graph replay")
    w = workloads.decode_inputs(16, seed=31, device=gpu, gate="slow", state_scale=0.5)
    out = torch.empty_like(w["v"])
    ns = torch.empty_like(w["state"])

    def step():
        binding.decode_kernel(w["q"], w["k"], w["v"], w["state"], w["A_log"], w["a"],
                              w["dt_bias"], w["b"], w["scale"], out, ns)

    step()
    torch.cuda.synchronize()
    ref_o, ref_s = out.clone(), ns.clone()
    g = _capture(step)
    for rep in range(4):
        out.fill_(float("nan"))
        ns.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_o), f"replay {rep}: output differs"
        assert torch.equal(ns, ref_s), f"replay {rep}: state differs"
        x = torch.randn(1 << 20, device=gpu).sum()        # unrelated eager work in between
        assert torch.isfinite(x)


@pytest.mark.parametrize("path", ["drop-in", "workspace", "no-alloc"])
@pytest.mark.parametrize("lens", [[130, 3, 0, 64], [300], [2500]])
def test_prefill_graph_replays_match_eager(gpu, lens, path):
    """128 chains (one kernel) and 32 chains (split 8 ways), through the drop-in kernel
    (gdn_prefill), with a preallocated workspace (two kernels for 32 chains), and through
    gdn_prefill_no_alloc (two kernels in the library's scratch, nothing allocated during
    capture).  One 2,500-token sequence through the drop-in runs two kernels in the
    drop-in scratch when eager and one kernel when captured; both give the same bits."""
    say(f"prefill graph replay lens={lens} path={path}")
    p = workloads.prefill_inputs(lens, seed=32, device=gpu, gate="slow", state_scale=0.5)
    T, N = p["q"].shape[0], len(p["lengths"])
    out = torch.empty((T, 32, 128), dtype=torch.bfloat16, device=gpu)
    ns = torch.empty((N, 32, 128, 128), dtype=torch.float32, device=gpu)
    args = (p["q"], p["k"], p["v"], p["state"], p["A_log"], p["a"], p["dt_bias"], p["b"],
            p["cu_seqlens"], p["scale"], out, ns)
    if path == "drop-in":
        def step():
            binding.prefill_kernel(*args)
    elif path == "workspace":
        ws = torch.empty(binding.prefill_workspace_bytes(N, T, 32), dtype=torch.uint8, device=gpu)

        def step():
            binding.prefill_kernel_with_workspace(*args, ws)
    else:
        lib = _lib.load()
        ptr = lambda t: None if t is None else t.data_ptr()
        cargs = [ptr(p[k]) for k in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")]
        cargs += [p["cu_seqlens"].data_ptr(), _lib.GDN_INDEX_INT32, N, T, p["scale"], ptr(out),
                  ptr(ns), 16, 16, 32, 128, 128]

        def step():
            _lib.check(lib.gdn_prefill_no_alloc(*cargs, torch.cuda.current_stream().cuda_stream))

    binding.prefill_kernel(*args)                            # the drop-in's result is the reference
    torch.cuda.synchronize()
    ref_o, ref_s = out.clone(), ns.clone()
    g = _capture(step)
    for rep in range(3):
        out.zero_()
        ns.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref_o), f"replay {rep}: output differs"
        assert torch.equal(ns, ref_s), f"replay {rep}: state differs"
        step()                                               # eager call between replays
        torch.cuda.synchronize()
