"""Seeded synthetic inputs for the GDN decode / prefill workloads.

Distributions follow the benchmark configurations of this path: q, k bf16 randn
L2-normalised per head (normalised in fp32, then cast); v, a, b bf16 randn;
A_log = log U[1, 16]; dt_bias = 0.1 randn; scale = 1/sqrt(128); initial state
0.05 randn.  ``gate="slow"`` is a stress distribution with slow decay
(A_log = log U[0.01, 0.05], g ~ 0.97-0.99) and smaller beta, so that the state
path (the g*S term, inter-chunk propagation) dominates the outputs -- under the
default gates one 64-token chunk decays the state by e^-50 or more.
``gate="edge"`` drives the gate prologue's branches: softplus arguments above 20,
saturated beta and A_log from no decay at all to a state wiped every token.

All tensors are generated with a seeded ``torch.Generator`` on ``device``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

HQ, HK, HV, D = 16, 16, 32, 128


@dataclass
class Heads:
    hq: int = HQ
    hk: int = HK
    hv: int = HV
    dk: int = D
    dv: int = D


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _unit_bf16(shape, gen, device) -> torch.Tensor:
    x = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    x = x / x.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    return x.to(torch.bfloat16)


# A_log per v-head under gate="edge", cycled over the heads: no decay at all
# (exp(A_log) ~ 6e-6, g = 1 to fp32 precision), slow, moderate, the top of the
# baseline range (log 16) and beyond it (e^4 ~ 55: the state is wiped each token).
EDGE_A_LOG = (-12.0, -4.0, 0.0, math.log(16.0), 4.0)


def _params(hv: int, gate: str, gen, device):
    if gate == "edge":
        A_log = torch.tensor([EDGE_A_LOG[h % len(EDGE_A_LOG)] for h in range(hv)],
                             dtype=torch.float32, device=device)
        dt_bias = 0.1 * torch.randn(hv, generator=gen, device=device, dtype=torch.float32)
        return A_log, dt_bias
    if gate == "baseline":
        lo, hi = 1.0, 16.0
    elif gate == "slow":
        lo, hi = 0.01, 0.05
    else:
        raise ValueError(f"unknown gate distribution {gate!r}")
    u = torch.rand(hv, generator=gen, device=device, dtype=torch.float32)
    A_log = torch.log(lo + (hi - lo) * u)
    dt_bias = 0.1 * torch.randn(hv, generator=gen, device=device, dtype=torch.float32)
    return A_log, dt_bias


def _edge_ab(shape, gen, device):
    """Gate inputs a, b for gate="edge": a mixes N(0,1) with values in [21, 40]
    (softplus takes its linear branch, x > 20) and with -40 (softplus ~ 4e-18);
    b mixes N(0,1) with +-12 (beta saturates at 1 - 6e-6 and 6e-6) and +-30."""
    u = torch.rand(shape, generator=gen, device=device)
    a = torch.randn(shape, generator=gen, device=device)
    a = torch.where(u < 0.35, 21.0 + 19.0 * torch.rand(shape, generator=gen, device=device), a)
    a = torch.where((u >= 0.35) & (u < 0.45), torch.full_like(a, -40.0), a)
    w = torch.rand(shape, generator=gen, device=device)
    b = torch.randn(shape, generator=gen, device=device)
    sgn = torch.where(torch.rand(shape, generator=gen, device=device) < 0.5, -1.0, 1.0)
    b = torch.where(w < 0.3, 12.0 * sgn, b)
    b = torch.where((w >= 0.3) & (w < 0.4), 30.0 * sgn, b)
    return a.to(torch.bfloat16), b.to(torch.bfloat16)


def decode_inputs(batch: int, heads: Heads = Heads(), seed: int = 0, device="cpu",
                  gate: str = "baseline", state_scale: float = 0.05, with_state: bool = True,
                  pool_slots: int | None = None) -> dict:
    """Inputs of one decode step.  With ``pool_slots`` the state is a pool of
    that many slots and ``state_indices`` is a random permutation prefix (int32,
    distinct)."""
    gen = _gen(seed, device)
    B, h = batch, heads
    out = {
        "q": _unit_bf16((B, 1, h.hq, h.dk), gen, device),
        "k": _unit_bf16((B, 1, h.hk, h.dk), gen, device),
        "v": torch.randn((B, 1, h.hv, h.dv), generator=gen, device=device).to(torch.bfloat16),
    }
    out["A_log"], out["dt_bias"] = _params(h.hv, gate, gen, device)
    if gate == "edge":
        out["a"], out["b"] = _edge_ab((B, 1, h.hv), gen, device)
    else:
        out["a"] = torch.randn((B, 1, h.hv), generator=gen, device=device).to(torch.bfloat16)
        bshift = -1.0 if gate == "slow" else 0.0
        out["b"] = (torch.randn((B, 1, h.hv), generator=gen, device=device) + bshift).to(torch.bfloat16)
    out["scale"] = 1.0 / math.sqrt(h.dk)
    nstate = pool_slots if pool_slots is not None else B
    if with_state or pool_slots is not None:
        out["state"] = state_scale * torch.randn((nstate, h.hv, h.dv, h.dk), generator=gen,
                                                 device=device, dtype=torch.float32)
    else:
        out["state"] = None
    if pool_slots is not None:
        if batch > pool_slots:
            raise ValueError("batch exceeds pool_slots")
        perm = torch.randperm(pool_slots, generator=gen, device=device)[:batch]
        out["state_indices"] = perm.to(torch.int32)
    return out


def varlen_lengths(num_seqs: int, total: int, max_len: int = 4096, seed: int = 4,
                   require_short: bool = True) -> list[int]:
    """Sequence lengths drawn log-uniform in [1, max_len], rescaled to sum to
    ``total``, rounded, clamped >= 1, rounding residue put on the longest;
    redrawn (next seed) until at least one length is shorter than one 64-token
    chunk when ``require_short``."""
    s = seed
    while True:
        rng = np.random.default_rng(s)
        raw = np.exp(rng.uniform(0.0, math.log(max_len), size=num_seqs))
        lens = np.maximum(1, np.round(raw * total / raw.sum())).astype(np.int64)
        lens[np.argmax(lens)] += total - int(lens.sum())
        if lens.min() >= 1 and (not require_short or lens.min() < 64):
            return [int(x) for x in lens]
        s += 1000


def prefill_inputs(lengths, heads: Heads = Heads(), seed: int = 0, device="cpu",
                   gate: str = "baseline", state_scale: float = 0.05, with_state: bool = True,
                   cu_dtype=torch.int32) -> dict:
    """Packed varlen prefill inputs for sequences of the given lengths."""
    gen = _gen(seed, device)
    h = heads
    lengths = [int(x) for x in lengths]
    T = int(sum(lengths))
    N = len(lengths)
    out = {
        "q": _unit_bf16((T, h.hq, h.dk), gen, device),
        "k": _unit_bf16((T, h.hk, h.dk), gen, device),
        "v": torch.randn((T, h.hv, h.dv), generator=gen, device=device).to(torch.bfloat16),
    }
    out["A_log"], out["dt_bias"] = _params(h.hv, gate, gen, device)
    if gate == "edge":
        out["a"], out["b"] = _edge_ab((T, h.hv), gen, device)
    else:
        out["a"] = torch.randn((T, h.hv), generator=gen, device=device).to(torch.bfloat16)
        bshift = -1.0 if gate == "slow" else 0.0
        out["b"] = (torch.randn((T, h.hv), generator=gen, device=device) + bshift).to(torch.bfloat16)
    out["scale"] = 1.0 / math.sqrt(h.dk)
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    out["cu_seqlens"] = torch.tensor(cu, dtype=cu_dtype, device=device)
    out["lengths"] = lengths
    if with_state:
        out["state"] = state_scale * torch.randn((N, h.hv, h.dv, h.dk), generator=gen,
                                                 device=device, dtype=torch.float32)
    else:
        out["state"] = None
    return out


# The benchmark configurations (decode B=1 CPU; decode B=64; pooled decode B=512 over
# 1024 slots; prefill T=4096 single sequence; prefill 32 sequences / 32768 tokens).
CONFIG4_NUM_SEQS = 32
CONFIG4_TOTAL = 32768


def config(idx: int, device="cpu", seed: int | None = None) -> dict:
    seed = idx if seed is None else seed
    if idx == 0:
        return decode_inputs(1, seed=seed, device=device)
    if idx == 1:
        return decode_inputs(64, seed=seed, device=device)
    if idx == 2:
        return decode_inputs(512, seed=seed, device=device, pool_slots=1024)
    if idx == 3:
        return prefill_inputs([4096], seed=seed, device=device, with_state=False)
    if idx == 4:
        return prefill_inputs(varlen_lengths(CONFIG4_NUM_SEQS, CONFIG4_TOTAL), seed=seed,
                              device=device)
    raise ValueError(f"no config {idx}")


def to_numpy(t):
    """float64 numpy copy of a tensor (bf16 values are exact in float64)."""
    if t is None:
        return None
    return t.detach().to("cpu", torch.float64).numpy()
