"""GPU parity tests of the decode kernel (through the C ABI) against the CPU oracle."""
import numpy as np
import pytest
import torch

from gdn_kernel_amd import _lib, binding, workloads
from gdn_kernel_amd.workloads import Heads, to_numpy
from oracle import gdn_oracle as O
from tests.conftest import assert_close
from tests.gpu_util import (OUT_ATOL, OUT_RTOL, STATE_ATOL, STATE_RTOL, host, oracle_decode,
                            run_decode, say)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B", [1, 3, 8])
@pytest.mark.parametrize("gate", ["baseline", "slow"])
@pytest.mark.parametrize("mode", ["in_place", "separate", "null_state"])
def test_decode_matches_oracle(gpu, B, gate, mode):
    say(f"decode parity B={B} gate={gate} mode={mode}")
    w = workloads.decode_inputs(B, seed=100 + B, gate=gate, with_state=mode != "null_state",
                                state_scale=1.0 if gate == "slow" else 0.05)
    o_ref, s_ref = oracle_decode(w)
    out, ns = run_decode(w, gpu, in_place=mode == "in_place")
    torch.cuda.synchronize()
    assert_close(host(out), o_ref, OUT_RTOL, OUT_ATOL, "output")
    assert_close(host(ns), s_ref, STATE_RTOL, STATE_ATOL, "new_state")


@pytest.mark.parametrize("hq,hk,hv", [(8, 8, 32), (4, 16, 32), (32, 32, 32), (1, 1, 4)])
def test_decode_head_ratios(gpu, hq, hk, hv):
    say(f"decode heads hq={hq} hk={hk} hv={hv}")
    w = workloads.decode_inputs(4, Heads(hq, hk, hv), seed=7, gate="slow", state_scale=0.5)
    o_ref, s_ref = oracle_decode(w)
    out, ns = run_decode(w, gpu, in_place=False)
    torch.cuda.synchronize()
    assert_close(host(out), o_ref, OUT_RTOL, OUT_ATOL, "output")
    assert_close(host(ns), s_ref, STATE_RTOL, STATE_ATOL, "new_state")


def test_decode_scale_argument(gpu):
    say("decode scale 0 / None / explicit")
    w = workloads.decode_inputs(2, seed=3)
    o_def, _ = run_decode(w, gpu, in_place=False)
    o_none, _ = run_decode({**w, "scale": None}, gpu, in_place=False)
    o_zero, _ = run_decode({**w, "scale": 0.0}, gpu, in_place=False)
    o_half, _ = run_decode({**w, "scale": 0.5}, gpu, in_place=False)
    torch.cuda.synchronize()
    assert torch.equal(o_def, o_none) and torch.equal(o_def, o_zero)
    ref, _ = O.decode(*[to_numpy(w[k]) for k in ("q", "k", "v", "state", "A_log", "a",
                                                  "dt_bias", "b")], 0.5)
    assert_close(host(o_half), ref, OUT_RTOL, OUT_ATOL, "output scale 0.5")


def test_decode_config1_full_size(gpu):
    """BASELINE config 1 (B=64, heads 16/16/32, state updated in place) vs the oracle."""
    say("decode config1 B=64 full size")
    w = workloads.config(1)
    o_ref, s_ref = oracle_decode(w)
    out, ns = run_decode(w, gpu, in_place=True)
    torch.cuda.synchronize()
    assert_close(host(out), o_ref, OUT_RTOL, OUT_ATOL, "output")
    assert_close(host(ns), s_ref, STATE_RTOL, STATE_ATOL, "new_state")


def test_decode_deterministic_and_alias_safe(gpu):
    say("decode determinism / aliasing")
    w = workloads.decode_inputs(16, seed=5, gate="slow", state_scale=0.5)
    o1, s1 = run_decode(w, gpu, in_place=False)
    o2, s2 = run_decode(w, gpu, in_place=True)       # fresh device copy updated in place
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(s1, s2)


def test_decode_empty_batch(gpu):
    say("decode B=0")
    w = workloads.decode_inputs(0, seed=1)
    out, ns = run_decode(w, gpu, in_place=True)
    torch.cuda.synchronize()
    assert out.numel() == 0


@pytest.mark.parametrize("gate", ["baseline", "slow"])
@pytest.mark.parametrize("B", [12, 8])
def test_decode_pooled_matches_oracle(gpu, gate, B):
    """Pooled decode with padding rows against the oracle, at B = 12 and B = 8 over
    40 slots."""
    say(f"decode pooled small gate={gate} B={B}")
    slots = 40
    w = workloads.decode_inputs(B, seed=9, gate=gate, pool_slots=slots,
                                state_scale=1.0 if gate == "slow" else 0.05)
    idx = w["state_indices"].clone()
    idx[3] = -1                      # padding row
    idx[7] = slots + 5               # out of range: treated as padding
    d = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    pool = d["state"].clone()
    out = torch.full_like(d["v"], float("nan"))
    binding.decode_pooled_kernel(d["q"], d["k"], d["v"], pool, d["A_log"], d["a"], d["dt_bias"],
                                 d["b"], d["scale"], out, idx.to(gpu))
    torch.cuda.synchronize()
    o_ref, pool_ref = O.decode_pooled(*[to_numpy(w[k]) for k in ("q", "k", "v", "state")],
                                      idx.numpy(), *[to_numpy(w[k]) for k in
                                                     ("A_log", "a", "dt_bias", "b")], w["scale"])
    assert_close(host(out), o_ref, OUT_RTOL, OUT_ATOL, "output")
    assert not host(out)[[3, 7]].any()
    assert_close(host(pool), pool_ref, STATE_RTOL, STATE_ATOL, "pool")
    used = set(int(i) for i in idx.tolist() if 0 <= i < slots)
    untouched = [s for s in range(slots) if s not in used]
    assert torch.equal(pool[untouched], d["state"][untouched]), "untouched slots changed"


def test_decode_pooled_more_rows_than_slots(gpu):
    """24 rows over 10 slots: rows 0-9 name every slot once, rows 10-23 are padding
    (negative or past the pool) with zero output."""
    say("decode pooled: 24 rows over 10 slots")
    slots, B = 10, 24
    w = workloads.decode_inputs(B, seed=77, gate="slow", pool_slots=24, state_scale=1.0)
    pool0 = w["state"][:slots].clone()
    idx = torch.cat([torch.randperm(slots, generator=torch.Generator().manual_seed(5)).to(torch.int32),
                     torch.tensor([-1, 10, 11, -7, 40, 12, -1, 99, 10, 13, -2, 1000, 15, -3],
                                  dtype=torch.int32)])
    o_ref, pool_ref = O.decode_pooled(*[to_numpy(w[k]) for k in ("q", "k", "v")], to_numpy(pool0),
                                      idx.numpy(), *[to_numpy(w[k]) for k in
                                                     ("A_log", "a", "dt_bias", "b")], w["scale"])
    d = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    pool = pool0.to(gpu)
    out = torch.full_like(d["v"], float("nan"))
    binding.decode_pooled_kernel(d["q"], d["k"], d["v"], pool, d["A_log"], d["a"], d["dt_bias"],
                                 d["b"], d["scale"], out, idx.to(gpu))
    torch.cuda.synchronize()
    assert not host(out)[10:].any()
    assert_close(host(out), o_ref, OUT_RTOL, OUT_ATOL, "output")
    assert_close(host(pool), pool_ref, STATE_RTOL, STATE_ATOL, "pool")


def test_decode_pooled_config2_full_size(gpu):
    """BASELINE config 2 (B=512 over a 1024-slot pool): every output row and every touched
    slot against the oracle (gather -> decode -> scatter); untouched slots bit-identical;
    touched slots equal the contiguous decode kernel on the gathered states."""
    say("decode pooled config2 full size")
    w = workloads.decode_inputs(512, seed=2, pool_slots=1024)
    o_ref, pool_ref = O.decode_pooled(*[to_numpy(w[k]) for k in ("q", "k", "v", "state")],
                                      w["state_indices"].numpy(),
                                      *[to_numpy(w[k]) for k in ("A_log", "a", "dt_bias", "b")],
                                      w["scale"])
    w = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    idx = w["state_indices"]
    pool = w["state"].clone()
    out = torch.empty_like(w["v"])
    binding.decode_pooled_kernel(w["q"], w["k"], w["v"], pool, w["A_log"], w["a"], w["dt_bias"],
                                 w["b"], w["scale"], out, idx)
    gathered = w["state"][idx.long()]
    out2 = torch.empty_like(w["v"])
    binding.decode_kernel(w["q"], w["k"], w["v"], gathered, w["A_log"], w["a"], w["dt_bias"],
                          w["b"], w["scale"], out2, gathered)
    torch.cuda.synchronize()
    assert_close(host(out), o_ref, OUT_RTOL, OUT_ATOL, "output")
    assert_close(host(pool), pool_ref, STATE_RTOL, STATE_ATOL, "pool")
    mask = torch.ones(1024, dtype=torch.bool, device=gpu)
    mask[idx.long()] = False
    assert torch.equal(pool[mask], w["state"][mask])
    assert torch.equal(out, out2)
    assert torch.equal(pool[idx.long()], gathered)


@pytest.mark.conflicts_expected
@pytest.mark.parametrize("heads,B,slots", [((16, 16, 32), 12, 40), ((16, 16, 32), 8, 40),
                                           ((1, 1, 4), 20, 64), ((1, 1, 4), 1500, 2048),
                                           ((1, 1, 4), 1500, 8000)])
def test_decode_pooled_duplicate_slots(gpu, heads, B, slots):
    """Rows naming a slot that another row also names: a pair at the first and last row
    (the two ends of the index scan), a triple in the middle, plus a padding row.  Each
    conflicting row has zero output and its slot keeps its bits; every other row matches
    the oracle; gdn_decode_pool_conflicts counts the five skipped rows.  The layouts take
    one-wave (B*Hv < 128) and four-wave workgroups, over several scan passes for B = 1500,
    and pools of 3 to 5 slots per row."""
    say(f"decode pooled duplicate slots heads={heads} B={B} slots={slots}")
    w = workloads.decode_inputs(B, Heads(*heads), seed=40 + B, gate="slow", pool_slots=slots,
                                state_scale=1.0)
    idx = w["state_indices"].clone()
    mid = B // 2
    idx[B - 1] = idx[0]
    idx[mid + 1] = idx[mid]
    idx[mid + 2] = idx[mid]
    idx[1] = -1
    conflict = O.pool_conflicts(idx.numpy(), slots)
    assert int(conflict.sum()) == 5
    o_ref, pool_ref = O.decode_pooled(*[to_numpy(w[k]) for k in ("q", "k", "v", "state")],
                                      idx.numpy(), *[to_numpy(w[k]) for k in
                                                     ("A_log", "a", "dt_bias", "b")], w["scale"])
    d = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in w.items()}
    pool = d["state"].clone()
    out = torch.full_like(d["v"], float("nan"))
    binding.decode_pool_conflicts(reset=True)
    binding.decode_pooled_kernel(d["q"], d["k"], d["v"], pool, d["A_log"], d["a"], d["dt_bias"],
                                 d["b"], d["scale"], out, idx.to(gpu))
    assert binding.decode_pool_conflicts(reset=True) == 5
    assert not host(out)[conflict].any()
    assert_close(host(out), o_ref, OUT_RTOL, OUT_ATOL, "output")
    shared = sorted(set(int(i) for i in idx[torch.from_numpy(conflict)].tolist()))
    assert torch.equal(pool[shared], d["state"][shared]), "a conflicting slot was written"
    assert_close(host(pool), pool_ref, STATE_RTOL, STATE_ATOL, "pool")


@pytest.mark.parametrize("B", [1, 8])
def test_decode_edge_gates(gpu, B):
    """The gate prologue's edge branches against the oracle: softplus arguments above 20,
    saturated beta (b = +-12, +-30) and A_log from -12 (no decay) to 4, per v-head."""
    say(f"decode edge gates B={B}")
    w = workloads.decode_inputs(B, seed=42, gate="edge", state_scale=0.5)
    x = to_numpy(w["a"]) + to_numpy(w["dt_bias"])
    assert (x > 20).any()
    o_ref, s_ref = oracle_decode(w)
    out, ns = run_decode(w, gpu, in_place=False)
    torch.cuda.synchronize()
    assert_close(host(out), o_ref, OUT_RTOL, OUT_ATOL, "output")
    assert_close(host(ns), s_ref, STATE_RTOL, STATE_ATOL, "new_state")


def test_decode_golden_fixture(gpu):
    say("decode golden fixture")
    fx = np.load(__import__("tests.golden", fromlist=["x"]).path("decode_small.npz"))
    t = lambda a, dt: torch.from_numpy(a).to(gpu).view(dt) if a.dtype == np.uint16 \
        else torch.from_numpy(a).to(gpu)
    q, k, v = (t(fx[n], torch.bfloat16) for n in ("q", "k", "v"))
    a, b = t(fx["a"], torch.bfloat16), t(fx["b"], torch.bfloat16)
    state = torch.from_numpy(O.bits_to_f32(fx["state"])).to(gpu)
    out = torch.empty_like(v)
    ns = torch.empty_like(state)
    binding.decode_kernel(q, k, v, state, t(fx["A_log"], None), a, t(fx["dt_bias"], None), b,
                          float(fx["scale"]), out, ns)
    torch.cuda.synchronize()
    assert_close(host(out), fx["out_ref"], OUT_RTOL, OUT_ATOL, "output")
    assert_close(host(ns), fx["state_ref"], STATE_RTOL, STATE_ATOL, "new_state")


def test_decode_every_launch_shape(gpu):
    """Every compiled decode launch shape (rows per wavefront x wavefronts per workgroup
    x nontemporal access), selected through gdn_decode_with_variant /
    gdn_decode_pooled_with_variant, against the oracle: in place, with a null state, and
    pooled with a padding row.  Production picks two of them by batch size."""
    lib = _lib.load()
    nv = lib.gdn_decode_num_variants()
    assert nv == 16
    stream = torch.cuda.current_stream(gpu).cuda_stream
    ptr = lambda t: None if t is None else t.data_ptr()
    w = workloads.decode_inputs(5, seed=31, gate="slow", state_scale=1.0)
    wn = workloads.decode_inputs(5, seed=32, gate="baseline", with_state=False)
    slots = 9
    wp = workloads.decode_inputs(4, seed=33, gate="slow", pool_slots=slots, state_scale=1.0)
    idx = wp["state_indices"].clone()
    idx[2] = -1
    o_ref, s_ref = oracle_decode(w)
    on_ref, sn_ref = oracle_decode(wn)
    op_ref, pool_ref = O.decode_pooled(*[to_numpy(wp[k]) for k in ("q", "k", "v", "state")],
                                       idx.numpy(), *[to_numpy(wp[k]) for k in
                                                      ("A_log", "a", "dt_bias", "b")], wp["scale"])
    H = (16, 16, 32, 128, 128)
    for variant in range(nv):
        say(f"decode launch shape {variant}")
        for ws, st_ref, ou_ref in ((w, s_ref, o_ref), (wn, sn_ref, on_ref)):
            d = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in ws.items()}
            out = torch.full_like(d["v"], float("nan"))
            ns = d["state"].clone() if d["state"] is not None else \
                torch.full((5, 32, 128, 128), float("nan"), device=gpu)
            st = ns if d["state"] is not None else None          # in place
            _lib.check(lib.gdn_decode_with_variant(
                ptr(d["q"]), ptr(d["k"]), ptr(d["v"]), ptr(st), ptr(d["A_log"]), ptr(d["a"]),
                ptr(d["dt_bias"]), ptr(d["b"]), d["scale"], ptr(out), ptr(ns), 5, *H, variant, stream))
            torch.cuda.synchronize()
            assert_close(host(out), ou_ref, OUT_RTOL, OUT_ATOL, f"shape {variant} output")
            assert_close(host(ns), st_ref, STATE_RTOL, STATE_ATOL, f"shape {variant} new_state")
        d = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in wp.items()}
        pool = d["state"].clone()
        out = torch.full_like(d["v"], float("nan"))
        _lib.check(lib.gdn_decode_pooled_with_variant(
            ptr(d["q"]), ptr(d["k"]), ptr(d["v"]), ptr(pool), slots, ptr(idx.to(gpu)), ptr(d["A_log"]),
            ptr(d["a"]), ptr(d["dt_bias"]), ptr(d["b"]), d["scale"], ptr(out), 4, *H, variant, stream))
        torch.cuda.synchronize()
        assert_close(host(out), op_ref, OUT_RTOL, OUT_ATOL, f"shape {variant} pooled output")
        assert_close(host(pool), pool_ref, STATE_RTOL, STATE_ATOL, f"shape {variant} pool")


@pytest.mark.conflicts_expected
@pytest.mark.parametrize("slots", [11, 30])
def test_decode_pooled_duplicates_every_launch_shape(gpu, slots):
    """Every compiled launch shape on a pooled batch of 5 rows whose rows 0 and 3 share a
    slot: both rows skipped (zero output, slot bit-identical), the others against the
    oracle, and two conflicts counted per launch, over pools of 11 and 30 slots."""
    lib = _lib.load()
    stream = torch.cuda.current_stream(gpu).cuda_stream
    ptr = lambda t: None if t is None else t.data_ptr()
    wp = workloads.decode_inputs(5, seed=34, gate="slow", pool_slots=slots, state_scale=1.0)
    idx = wp["state_indices"].clone()
    idx[3] = idx[0]
    op_ref, pool_ref = O.decode_pooled(*[to_numpy(wp[k]) for k in ("q", "k", "v", "state")],
                                       idx.numpy(), *[to_numpy(wp[k]) for k in
                                                      ("A_log", "a", "dt_bias", "b")], wp["scale"])
    H = (16, 16, 32, 128, 128)
    d = {k: (v.to(gpu) if isinstance(v, torch.Tensor) else v) for k, v in wp.items()}
    binding.decode_pool_conflicts(reset=True)
    for variant in range(lib.gdn_decode_num_variants()):
        say(f"decode pooled duplicates, {slots} slots, launch shape {variant}")
        pool = d["state"].clone()
        out = torch.full_like(d["v"], float("nan"))
        _lib.check(lib.gdn_decode_pooled_with_variant(
            ptr(d["q"]), ptr(d["k"]), ptr(d["v"]), ptr(pool), slots, ptr(idx.to(gpu)), ptr(d["A_log"]),
            ptr(d["a"]), ptr(d["dt_bias"]), ptr(d["b"]), d["scale"], ptr(out), 5, *H, variant, stream))
        assert binding.decode_pool_conflicts(reset=True) == 2, f"shape {variant}"
        assert not host(out)[[0, 3]].any()
        assert_close(host(out), op_ref, OUT_RTOL, OUT_ATOL, f"shape {variant} pooled output")
        assert torch.equal(pool[int(idx[0])], d["state"][int(idx[0])])
        assert_close(host(pool), pool_ref, STATE_RTOL, STATE_ATOL, f"shape {variant} pool")


def test_decode_max_heads(gpu):
    """The largest head count the C ABI accepts (GDN_MAX_HEADS = 65,536 q, k and v heads),
    B = 2, state updated in place: every output element is written, and five heads at
    both ends and in the middle match the oracle run on those heads alone."""
    h = _lib.GDN_MAX_HEADS
    say(f"decode max heads Hq=Hk=Hv={h} B=2")
    w = workloads.decode_inputs(2, Heads(h, h, h), seed=78, device=gpu, gate="slow", state_scale=0.5)
    gi = torch.tensor([0, 1, h // 2 + 3, h - 2, h - 1], device=gpu)
    sub = {k: w[k][:, :, gi].cpu() for k in ("q", "k", "v", "a", "b")}
    sub.update({k: w[k][gi].cpu() for k in ("A_log", "dt_bias")})
    sub["state"], sub["scale"] = w["state"][:, gi].cpu(), w["scale"]
    out, ns = run_decode(w, gpu, in_place=True)
    torch.cuda.synchronize()
    assert not torch.isnan(out).any()
    o_ref, s_ref = oracle_decode(sub)
    assert_close(host(out[:, :, gi]), o_ref, OUT_RTOL, OUT_ATOL, "output")
    assert_close(host(ns[:, gi]), s_ref, STATE_RTOL, STATE_ATOL, "new_state")
