"""PyTorch float32 implementations of the two GDN definitions, for the trace runner.

These are the "reference" side of a FlashInfer-Bench evaluation: the runner
(``gdn_kernel_amd.bench_runner``) computes ground-truth outputs with them and
times them as ``reference_latency_ms``.  They are never called by the kernel
entry points (``gdn_kernel_amd.binding``), which run only the HIP library.

* ``decode_reference`` follows the decode definition's ``run``
  (/root/reference/design.md:166-226): g = exp(-exp(A_log) softplus(a + dt_bias)),
  beta = sigmoid(b), old_state = g S, old_v = k old_state,
  new_v = beta v + (1 - beta) old_v, S' = old_state - k (x) old_v + k (x) new_v,
  o = scale q S'; heads are read from the shapes, v-head h uses qk-head
  h // (Hv / Hq) (design.md:137-146, 199-200).
* ``prefill_reference`` is the chunked form of the sequential definition
  (prefill_design.md:497-545) over packed varlen sequences
  (solution/cuda/kernel_prefill.cu:46, 56-66): per 64-token chunk,
  T~ = (I + strictLower(beta Gamma KK^T))^-1 by forward substitution, then
  v_new = T~ (beta V) - T~ (beta e^gamma K) S^T, o = scale (e^gamma Q S^T +
  tril(Gamma QK^T) v_new), S = e^{gamma_last} S + v_new^T (K e^{gamma_last - gamma})
  (kernel_prefill.cu:95-294).  It equals the token-by-token definition in exact
  arithmetic (checked against the CPU oracle in tests/test_bench_runner.py).

All arithmetic is float32 on the tensors' device; outputs are returned as bf16,
new states as float32.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = ["decode_reference", "prefill_reference"]


def _scale(scale, dk: int) -> float:
    if scale is None or float(scale) == 0.0:
        return 1.0 / math.sqrt(dk)
    return float(scale)


def _log_gates(A_log, a, dt_bias, b):
    x = a.float() + dt_bias.float()
    lg = -torch.exp(A_log.float()) * F.softplus(x)       # softplus threshold 20 (torch default)
    return lg, torch.sigmoid(b.float())


@torch.no_grad()
def decode_reference(q, k, v, state, A_log, a, dt_bias, b, scale):
    """q,k [B,1,H{q,k},K]; v [B,1,Hv,V]; state [B,Hv,V,K] or None; a,b [B,1,Hv].
    Returns (output [B,1,Hv,V] bf16, new_state [B,Hv,V,K] fp32)."""
    B, _, Hq, K = q.shape
    Hk, Hv, V = k.shape[2], v.shape[2], v.shape[3]
    scale = _scale(scale, K)
    lg, beta = _log_gates(A_log, a[:, 0], dt_bias, b[:, 0])        # [B,Hv]
    g = torch.exp(lg)
    qe = q[:, 0].float().repeat_interleave(Hv // Hq, dim=1)        # [B,Hv,K]
    ke = k[:, 0].float().repeat_interleave(Hv // Hk, dim=1)
    vv = v[:, 0].float()                                           # [B,Hv,V]
    S = (torch.zeros(B, Hv, V, K, device=q.device) if state is None
         else state.float()) * g[..., None, None]                  # old_state, k-last
    old_v = torch.einsum("bhvk,bhk->bhv", S, ke)
    new_v = beta[..., None] * vv + (1 - beta[..., None]) * old_v
    S = S + (new_v - old_v)[..., :, None] * ke[..., None, :]
    out = scale * torch.einsum("bhvk,bhk->bhv", S, qe)
    return out[:, None].to(torch.bfloat16), S


def _unit_lower_inverse(N):
    """(I + N)^-1 for strictly-lower N [..., C, C], row by row (kernel_prefill.cu:148-163)."""
    C = N.shape[-1]
    X = -N.clone()
    for i in range(1, C):
        X[..., i, :i] = X[..., i, :i] + (X[..., i, :i, None] * X[..., :i, :i]).sum(-2)
    return X + torch.eye(C, device=N.device, dtype=N.dtype)


@torch.no_grad()
def prefill_reference(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale, chunk: int = 64):
    """q,k [T,H{q,k},K]; v [T,Hv,V]; state [N,Hv,V,K] or None; a,b [T,Hv];
    cu_seqlens [N+1].  Returns (output [T,Hv,V] bf16, new_state [N,Hv,V,K] fp32)."""
    if q.dim() == 4:
        q, k, v, a, b = q[0], k[0], v[0], a[0], b[0]
    T, Hq, K = q.shape
    Hk, Hv, V = k.shape[1], v.shape[1], v.shape[2]
    scale = _scale(scale, K)
    dev = q.device
    lg, beta = _log_gates(A_log, a, dt_bias, b)                    # [T,Hv]
    cu = [int(x) for x in cu_seqlens.tolist()]
    N = len(cu) - 1
    S_all = (torch.zeros(N, Hv, V, K, device=dev) if state is None else state.float().clone())
    out = torch.zeros(T, Hv, V, device=dev)
    C = chunk
    tri_s = torch.tril(torch.ones(C, C, dtype=torch.bool, device=dev), -1)
    tri_i = torch.tril(torch.ones(C, C, dtype=torch.bool, device=dev))
    for n in range(N):
        s0, s1 = max(0, min(cu[n], T)), max(0, min(cu[n + 1], T))
        if s1 <= s0:
            continue                                               # passes its state through
        S = S_all[n]                                               # [Hv,V,K]
        for cs in range(s0, s1, C):
            cl = min(C, s1 - cs)
            Qc = torch.zeros(Hv, C, K, device=dev)
            Kc = torch.zeros(Hv, C, K, device=dev)
            Vc = torch.zeros(Hv, C, V, device=dev)
            Qc[:, :cl] = q[cs:cs + cl].float().repeat_interleave(Hv // Hq, dim=1).transpose(0, 1)
            Kc[:, :cl] = k[cs:cs + cl].float().repeat_interleave(Hv // Hk, dim=1).transpose(0, 1)
            Vc[:, :cl] = v[cs:cs + cl].float().transpose(0, 1)
            gam = torch.zeros(Hv, C, device=dev)
            bet = torch.zeros(Hv, C, device=dev)
            gam[:, :cl] = lg[cs:cs + cl].t()
            bet[:, :cl] = beta[cs:cs + cl].t()
            gam = gam.cumsum(-1)
            diff = torch.where(tri_i, gam[:, :, None] - gam[:, None, :], torch.zeros((), device=dev))
            Gam = torch.exp(diff)
            Nm = torch.where(tri_s, bet[:, :, None] * (Kc @ Kc.transpose(1, 2)) * Gam,
                             torch.zeros((), device=dev))
            Tt = _unit_lower_inverse(Nm)
            P = torch.where(tri_i, (Qc @ Kc.transpose(1, 2)) * Gam, torch.zeros((), device=dev))
            eg = torch.exp(gam)
            W = Tt @ (Kc * (bet * eg)[..., None])
            v_new = Tt @ (bet[..., None] * Vc) - W @ S.transpose(1, 2)
            o = scale * ((Qc * eg[..., None]) @ S.transpose(1, 2) + P @ v_new)
            out[cs:cs + cl] = o[:, :cl].transpose(0, 1)
            g_last = gam[:, cl - 1]
            Kd = Kc * torch.exp(g_last[:, None] - gam)[..., None]
            S = S * torch.exp(g_last)[:, None, None] + v_new.transpose(1, 2) @ Kd
        S_all[n] = S
    return out.to(torch.bfloat16), S_all
