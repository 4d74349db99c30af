"""The reference's PyTorch decode definition, restated for the CPU baseline.

TEST INFRASTRUCTURE ONLY, like the rest of ``oracle/``: only ``tests/`` and
``bench.py``'s ``cpu_baseline`` leg use it (as the timed CPU baseline), never the
product path.

``decode_definition`` is the PyTorch ``run`` of /root/reference/design.md:166-226,
step for step: fp32 gates and beta (:182-185), GQA expansion by
``repeat_interleave`` (:199-200), then a Python loop over (batch row, v-head) with
the per-head matrix form old_state = g S^T, old_v = k old_state,
new_v = beta v + (1 - beta) old_v, S^T' = old_state - k old_v^T + k new_v^T,
o = scale q S^T' (:205-223).  The only change is that the head counts come from
the tensor shapes instead of the asserts 4/4/8 (:173-176), so BASELINE config 0
(heads 16/16/32) runs.  tests/test_oracle.py pins it to the numpy oracle.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

__all__ = ["decode_definition"]


@torch.no_grad()
def decode_definition(q, k, v, state, A_log, a, dt_bias, b, scale):
    """q,k [B,1,H{q,k},128] bf16, v [B,1,Hv,128] bf16, state [B,Hv,V,K] fp32 or None,
    A_log/dt_bias [Hv] fp32, a/b [B,1,Hv] bf16.  Returns (output [B,1,Hv,V] bf16,
    new_state [B,Hv,V,K] fp32)."""
    B, T, num_q_heads, K = q.shape
    num_k_heads = k.shape[2]
    num_v_heads, V = v.shape[2], v.shape[3]
    assert T == 1 and num_v_heads % num_q_heads == 0 and num_v_heads % num_k_heads == 0
    if scale is None or scale == 0.0:
        scale = 1.0 / math.sqrt(K)
    x = a.float() + dt_bias.float()
    g = torch.exp(-torch.exp(A_log.float()) * F.softplus(x))
    beta = torch.sigmoid(b.float())
    q_f32, k_f32, v_f32 = q.squeeze(1).float(), k.squeeze(1).float(), v.squeeze(1).float()
    g_f32, beta_f32 = g.squeeze(1).float(), beta.squeeze(1).float()
    state_f32 = (state.float() if state is not None
                 else torch.zeros(B, num_v_heads, V, K, dtype=torch.float32, device=q.device))
    q_exp = q_f32.repeat_interleave(num_v_heads // num_q_heads, dim=1)
    k_exp = k_f32.repeat_interleave(num_v_heads // num_k_heads, dim=1)
    new_state = torch.zeros_like(state_f32)
    output = torch.zeros(B, num_v_heads, V, dtype=torch.float32, device=q.device)
    for bi in range(B):
        for h in range(num_v_heads):
            q_h, k_h, v_h = q_exp[bi, h], k_exp[bi, h], v_f32[bi, h]
            h_state = state_f32[bi, h].clone().transpose(-1, -2)       # [K, V]
            old_state = g_f32[bi, h] * h_state
            old_v = k_h @ old_state
            new_v = beta_f32[bi, h] * v_h + (1 - beta_f32[bi, h]) * old_v
            h_state = (old_state - k_h.unsqueeze(1) @ old_v.unsqueeze(0)
                       + k_h.unsqueeze(1) @ new_v.unsqueeze(0))
            output[bi, h] = scale * (q_h @ h_state)
            new_state[bi, h] = h_state.transpose(-1, -2)
    return output.unsqueeze(1).to(torch.bfloat16), new_state
