"""CPU oracle for the Gated DeltaNet (GDN) decode step and varlen chunked prefill.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (``gdn_kernel_amd``) may
import, call or execute this module.  Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or
the timed CPU baseline), never as the thing measured on the GPU.

This is a numpy restatement of the reference's own definitions of the op:

* decode      -- the PyTorch ``run`` in /root/reference/design.md:166-226, with
  the hard-coded head asserts (design.md:173-176) parameterised: heads come from
  the tensor shapes, GQA ratio = Hv/Hq (design.md:137-146).
* prefill     -- the sequential ``run_prefill`` in
  /root/reference/prefill_design.md:497-545, generalised from ``[B, T]`` to the
  packed varlen layout ``[T_tot, H, d]`` + ``cu_seqlens`` that the reference
  prefill kernel uses (solution/cuda/kernel_prefill.cu:46, 56-66, 93-97, 307).
* cross-check forms -- FLA ``naive_recurrent_gated_delta_rule``
  (prefill_design.md:709-760, log-space gate) and ``naive_chunk_gated_delta_rule``
  (prefill_design.md:763-880), plus the per-chunk algorithm of the reference CUDA
  prefill kernel (kernel_prefill.cu:95-294: T~ by forward substitution, masked
  QK^T, inter-chunk state propagation).

All arithmetic is done in the dtype passed (float64 by default, float32 to
mirror the reference's ``.float()`` arithmetic).  bf16 tensors are represented
as float arrays whose values are exactly representable in bf16; ``bf16_round``
is round-to-nearest-even, as ``tensor.to(torch.bfloat16)`` does.

Layouts (all k-last, design.md:56, 253-254):
  decode : q,k [B,1,Hq,K]  v [B,1,Hv,V]  state [B,Hv,V,K]  a,b [B,1,Hv]
  prefill: q,k [T,Hq,K]    v [T,Hv,V]    state [N,Hv,V,K]  a,b [T,Hv]
  A_log, dt_bias [Hv];  output like v;  cu_seqlens [N+1]
"""
from __future__ import annotations

import math

import numpy as np

__all__ = [
    "bf16_round", "bf16_bits", "bits_to_f32", "softplus", "gates", "log_gates",
    "default_scale", "decode", "decode_pooled", "prefill_sequential",
    "recurrent_fla", "chunk_fla", "prefill_chunked",
]


# ----------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even, NaN preserved)
# ----------------------------------------------------------------------------
def bf16_bits(x) -> np.ndarray:
    """float -> uint16 bf16 bit pattern, round-to-nearest-even."""
    u = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + np.uint32(0x7FFF) + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bits_to_f32(bits) -> np.ndarray:
    """uint16 bf16 bit pattern -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x) -> np.ndarray:
    """Round to the nearest bf16 value (RNE); returns float32."""
    return bits_to_f32(bf16_bits(x))


# ----------------------------------------------------------------------------
# Gate / beta prologue
# ----------------------------------------------------------------------------
def softplus(x):
    """torch.nn.functional.softplus with its default threshold 20: x if x > 20
    else log(1 + e^x).  Same cut as kernel.cu:51 and triton/kernel.py:29."""
    x = np.asarray(x)
    with np.errstate(over="ignore"):
        return np.where(x > 20, x, np.log1p(np.exp(np.minimum(x, 20))))


def gates(A_log, a, dt_bias, b, dtype=np.float64):
    """g = exp(-exp(A_log) * softplus(a + dt_bias)), beta = sigmoid(b).

    design.md:183-185 (definition), kernel.cu:44-53 (reference decode kernel).
    ``a``/``b`` have the head axis last; A_log/dt_bias broadcast over it.
    """
    x = np.asarray(a, dtype) + np.asarray(dt_bias, dtype)
    g = np.exp(-np.exp(np.asarray(A_log, dtype)) * softplus(x))
    with np.errstate(over="ignore"):
        beta = 1.0 / (1.0 + np.exp(-np.asarray(b, dtype)))
    return g.astype(dtype), beta.astype(dtype)


def log_gates(A_log, a, dt_bias, b, dtype=np.float64):
    """Log-space gate as the prefill kernel forms it: gamma_t = -exp(A_log) *
    softplus(a_t + dt_bias), beta_t = sigmoid(b_t)  (kernel_prefill.cu:101-115)."""
    x = np.asarray(a, dtype) + np.asarray(dt_bias, dtype)
    lg = -np.exp(np.asarray(A_log, dtype)) * softplus(x)
    with np.errstate(over="ignore"):
        beta = 1.0 / (1.0 + np.exp(-np.asarray(b, dtype)))
    return lg.astype(dtype), beta.astype(dtype)


def default_scale(scale, head_dim_k: int) -> float:
    """``scale is None or scale == 0`` -> 1/sqrt(K) (design.md:179-180,
    kernel.cu:115-118, kernel_prefill.cu:308-309)."""
    if scale is None or float(scale) == 0.0:
        return 1.0 / math.sqrt(head_dim_k)
    return float(scale)


# ----------------------------------------------------------------------------
# Decode (T = 1)
# ----------------------------------------------------------------------------
def decode(q, k, v, state, A_log, a, dt_bias, b, scale, dtype=np.float64):
    """Literal restatement of the reference decode definition (design.md:166-226).

    Returns (output [B,1,Hv,V] in ``dtype`` -- round with ``bf16_round`` to get
    the bf16 output the definition returns --, new_state [B,Hv,V,K]).
    """
    q = np.asarray(q, dtype); k = np.asarray(k, dtype); v = np.asarray(v, dtype)
    B, T, Hq, K = q.shape
    Hk = k.shape[2]
    Hv, V = v.shape[2], v.shape[3]
    assert T == 1 and k.shape[:2] == (B, 1) and v.shape[:2] == (B, 1)
    assert Hv % Hq == 0 and Hv % Hk == 0
    scale = default_scale(scale, K)

    g, beta = gates(A_log, a, dt_bias, b, dtype)          # [B,1,Hv]
    g = g[:, 0]; beta = beta[:, 0]                        # [B,Hv]
    if state is None:                                     # design.md:193-196
        S0 = np.zeros((B, Hv, V, K), dtype)
    else:
        S0 = np.asarray(state, dtype)
    # GQA: v-head h reads qk-head h // (Hv/Hq)  (repeat_interleave, design.md:199-200)
    q_exp = np.repeat(q[:, 0], Hv // Hq, axis=1)          # [B,Hv,K]
    k_exp = np.repeat(k[:, 0], Hv // Hk, axis=1)
    v0 = v[:, 0]                                          # [B,Hv,V]

    new_state = np.zeros_like(S0)
    out = np.zeros((B, Hv, V), dtype)
    for bi in range(B):
        for h in range(Hv):
            q_h, k_h, v_h = q_exp[bi, h], k_exp[bi, h], v0[bi, h]
            h_state = S0[bi, h].T.copy()                  # [K,V]
            old_state = g[bi, h] * h_state
            old_v = k_h @ old_state                       # [V]
            new_v = beta[bi, h] * v_h + (1 - beta[bi, h]) * old_v
            h_state = (old_state - np.outer(k_h, old_v) + np.outer(k_h, new_v))
            out[bi, h] = scale * (q_h @ h_state)
            new_state[bi, h] = h_state.T
    return out[:, None], new_state


def pool_conflicts(state_indices, pool_slots):
    """Rows of a pooled decode batch whose in-range slot another row also names."""
    idx = np.asarray(state_indices).astype(np.int64)
    valid = (idx >= 0) & (idx < pool_slots)
    if not valid.any():
        return np.zeros(idx.shape, bool)
    uniq, counts = np.unique(idx[valid], return_counts=True)
    return valid & np.isin(idx, uniq[counts > 1])


def decode_pooled(q, k, v, pool, state_indices, A_log, a, dt_bias, b, scale,
                  dtype=np.float64):
    """Decode over an indexed state pool: gather pool[idx[b]] -> decode ->
    scatter back.  No reference counterpart; the semantics
    are gather/decode/scatter.  Slots outside [0, pool_slots) are padding:
    their output rows are zero and no pool slot is touched.  A slot that more than
    one in-range row names is a conflict (updating it from each row would race):
    every row naming it is treated as padding.  Untouched slots keep their exact
    bits.  Returns (output, new_pool)."""
    pool = np.asarray(pool, dtype)
    idx = np.asarray(state_indices).astype(np.int64)
    valid = (idx >= 0) & (idx < pool.shape[0])
    if valid.any():
        uniq, counts = np.unique(idx[valid], return_counts=True)
        valid &= ~np.isin(idx, uniq[counts > 1])
    B = q.shape[0]
    Hv, V = v.shape[2], v.shape[3]
    out = np.zeros((B, 1, Hv, V), dtype)
    new_pool = pool.copy()
    if valid.any():
        sel = np.nonzero(valid)[0]
        o, ns = decode(np.asarray(q)[sel], np.asarray(k)[sel], np.asarray(v)[sel],
                       pool[idx[sel]], A_log, np.asarray(a)[sel], dt_bias,
                       np.asarray(b)[sel], scale, dtype)
        out[sel] = o
        new_pool[idx[sel]] = ns
    return out, new_pool


# ----------------------------------------------------------------------------
# Prefill: sequential definition (arbiter), packed varlen
# ----------------------------------------------------------------------------
def _seq_bounds(cu_seqlens):
    cu = np.asarray(cu_seqlens).astype(np.int64)
    return [(int(cu[i]), int(cu[i + 1])) for i in range(len(cu) - 1)]


def prefill_sequential(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale,
                       dtype=np.float64):
    """Token-by-token restatement of ``run_prefill`` (prefill_design.md:497-545)
    over packed varlen sequences (kernel_prefill.cu:56-66): sequence i covers
    tokens [cu[i], cu[i+1]); a sequence with length <= 0 passes its initial
    state through unchanged; ``state is None`` means zero initial states.

    Heads are vectorised; the per-head step is exactly the definition's
    old_state = g*S; old_v = k@old_state; new_v = beta*v + (1-beta)*old_v;
    S = old_state - k (x) old_v + k (x) new_v; o = scale * q@S.
    Returns (output [T,Hv,V], new_state [N,Hv,V,K]).
    """
    q = np.asarray(q, dtype); k = np.asarray(k, dtype); v = np.asarray(v, dtype)
    T, Hq, K = q.shape
    Hk = k.shape[1]
    Hv, V = v.shape[1], v.shape[2]
    scale = default_scale(scale, K)
    bounds = _seq_bounds(cu_seqlens)
    N = len(bounds)
    g, beta = gates(A_log, a, dt_bias, b, dtype)          # [T,Hv]
    S_all = (np.zeros((N, Hv, V, K), dtype) if state is None
             else np.asarray(state, dtype).copy())
    out = np.zeros((T, Hv, V), dtype)
    rq, rk = Hv // Hq, Hv // Hk
    for n, (s, e) in enumerate(bounds):
        if e - s <= 0:
            continue
        S = np.transpose(S_all[n], (0, 2, 1)).copy()      # [Hv,K,V]
        for t in range(s, e):
            q_h = np.repeat(q[t], rq, axis=0)             # [Hv,K]
            k_h = np.repeat(k[t], rk, axis=0)
            v_h = v[t]                                    # [Hv,V]
            old_state = g[t][:, None, None] * S
            old_v = np.einsum("hk,hkv->hv", k_h, old_state)
            new_v = beta[t][:, None] * v_h + (1 - beta[t][:, None]) * old_v
            S = (old_state - k_h[:, :, None] * old_v[:, None, :]
                 + k_h[:, :, None] * new_v[:, None, :])
            out[t] = scale * np.einsum("hk,hkv->hv", q_h, S)
        S_all[n] = np.transpose(S, (0, 2, 1))
    return out, S_all


# ----------------------------------------------------------------------------
# Cross-check forms (FLA naive recurrent / naive chunk), single sequence
# ----------------------------------------------------------------------------
def recurrent_fla(q, k, v, beta, log_g, scale=None, initial_state=None,
                  dtype=np.float64):
    """FLA ``naive_recurrent_gated_delta_rule`` (prefill_design.md:709-760).

    q,k [T,H,K], v [T,H,V], beta/log_g [T,H] (gate in log space),
    initial_state [H,K,V] (K-major, FLA convention).  Heads are already
    expanded (no GQA here).  Returns (o [T,H,V], S [H,K,V]).
    """
    q = np.asarray(q, dtype); k = np.asarray(k, dtype); v = np.asarray(v, dtype)
    beta = np.asarray(beta, dtype); log_g = np.asarray(log_g, dtype)
    T, H, K = q.shape
    V = v.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    h = (np.zeros((H, K, V), dtype) if initial_state is None
         else np.asarray(initial_state, dtype).copy())
    q = q * scale
    o = np.zeros((T, H, V), dtype)
    for i in range(T):
        h = h * np.exp(log_g[i])[:, None, None]
        b_v = v[i] - (h * k[i][:, :, None]).sum(-2)
        b_v = b_v * beta[i][:, None]
        h = h + k[i][:, :, None] * b_v[:, None, :]
        o[i] = np.einsum("hd,hdm->hm", q[i], h)
    return o, h


def _tri_inverse_unit_lower(N):
    """(I + N)^{-1} for strictly-lower N, by the forward substitution of
    prefill_design.md:847-851 / kernel_prefill.cu:148-163.  N: [..., C, C]."""
    C = N.shape[-1]
    X = -N.copy()
    for i in range(1, C):
        # row i: X[i,:i] = -N[i,:i] + sum_{m<i} (-N[i,m]) * X[m,:i]
        X[..., i, :i] = X[..., i, :i] + np.einsum(
            "...m,...mj->...j", X[..., i, :i], X[..., :i, :i])
    eye = np.eye(C, dtype=N.dtype)
    return X + eye


def chunk_fla(q, k, v, log_g, beta, chunk_size=64, scale=None,
              initial_state=None, dtype=np.float64):
    """FLA ``naive_chunk_gated_delta_rule`` (prefill_design.md:763-880).

    Same argument conventions as ``recurrent_fla``.  The sequence is zero-padded
    to a multiple of ``chunk_size``; padded positions have beta = 0 and log-gate
    0, so they change nothing.  Returns (o [T,H,V], S [H,K,V]).
    """
    q = np.asarray(q, dtype); k = np.asarray(k, dtype); v = np.asarray(v, dtype)
    beta = np.asarray(beta, dtype); log_g = np.asarray(log_g, dtype)
    BT = chunk_size
    T, H, K = q.shape
    V = v.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(K)
    pad = (BT - T % BT) % BT
    tr = lambda x: np.moveaxis(x, 0, 1)                  # [T,H,...] -> [H,T,...]
    q, k, v, beta, log_g = map(tr, (q, k, v, beta, log_g))
    if pad:
        q = np.pad(q, ((0, 0), (0, pad), (0, 0)))
        k = np.pad(k, ((0, 0), (0, pad), (0, 0)))
        v = np.pad(v, ((0, 0), (0, pad), (0, 0)))
        beta = np.pad(beta, ((0, 0), (0, pad)))
        log_g = np.pad(log_g, ((0, 0), (0, pad)))
    L = T + pad
    n = L // BT
    q = q * scale
    v = v * beta[..., None]
    k_beta = k * beta[..., None]
    rs = lambda x: x.reshape(H, n, BT, *x.shape[2:])
    q, k, v, k_beta = map(rs, (q, k, v, k_beta))
    decay = rs(log_g).cumsum(-1)                          # [H,n,BT]
    decay_exp = np.exp(decay)[..., None]
    diff = decay[..., :, None] - decay[..., None, :]
    L_mask = np.tril(np.exp(np.tril(diff)))
    upper_incl = np.triu(np.ones((BT, BT), bool), 0)
    attn = -(k_beta @ np.swapaxes(k, -1, -2)) * L_mask
    attn = np.where(upper_incl, 0.0, attn)
    Tt = _tri_inverse_unit_lower(-attn)                  # (I + N)^-1, N = -attn
    u = Tt @ v                                           # U~
    w = Tt @ (k_beta * decay_exp)                        # <-W
    S = (np.zeros((H, K, V), dtype) if initial_state is None
         else np.asarray(initial_state, dtype).copy())
    o = np.zeros((H, n, BT, V), dtype)
    upper_strict = np.triu(np.ones((BT, BT), bool), 1)
    for i in range(n):
        q_i, k_i, u_i = q[:, i], k[:, i], u[:, i]
        attn_i = np.where(upper_strict, 0.0,
                          (q_i @ np.swapaxes(k_i, -1, -2)) * L_mask[:, i])
        v_prime = w[:, i] @ S
        v_new = u_i - v_prime
        o_inter = (q_i * np.exp(decay[:, i])[..., None]) @ S
        o[:, i] = o_inter + attn_i @ v_new
        last = decay[:, i, -1]
        S = (S * np.exp(last)[:, None, None]
             + np.swapaxes(k_i * np.exp(last[:, None] - decay[:, i])[..., None],
                           -1, -2) @ v_new)
    o = o.reshape(H, L, V)[:, :T]
    return np.moveaxis(o, 0, 1), S


# ----------------------------------------------------------------------------
# Prefill: the reference kernel's per-chunk algorithm, packed varlen
# ----------------------------------------------------------------------------
def prefill_chunked(q, k, v, state, A_log, a, dt_bias, b, cu_seqlens, scale,
                    chunk=64, dtype=np.float64):
    """Per-chunk algorithm of the reference prefill kernel
    (kernel_prefill.cu:95-294), over packed varlen sequences, heads vectorised.

    Per chunk of clen <= C tokens (positions >= clen padded with zero K/Q/V,
    beta = 0 and log-gate 0, kernel_prefill.cu:102-114, 125-132):
      gamma   = inclusive cumsum of the log gate            (:118-122)
      A_ij    = -beta_i (k_i.k_j) e^{gamma_i-gamma_j}, i>j   (:134-146)
      T~      = forward substitution, unit diagonal          (:148-163)
      P_ij    = (q_i.k_j) e^{gamma_i-gamma_j}, j<=i          (:165-185)
      W       = T~ (K * beta * e^gamma)                      (:187-195)
      inter   = (Q e^gamma) S^T, corr = W S^T                (:216-245)
      v_new   = T~ (beta V) - corr                           (:251-271)
      o       = scale (inter + P v_new)                      (:273-283)
      S       = e^{gamma_last} S + v_new^T (K e^{gamma_last-gamma})  (:197-202, 286-293)
    Returns (output [T,Hv,V], new_state [N,Hv,V,K]).
    """
    q = np.asarray(q, dtype); k = np.asarray(k, dtype); v = np.asarray(v, dtype)
    T, Hq, K = q.shape
    Hk = k.shape[1]
    Hv, V = v.shape[1], v.shape[2]
    scale = default_scale(scale, K)
    bounds = _seq_bounds(cu_seqlens)
    N = len(bounds)
    lg, beta = log_gates(A_log, a, dt_bias, b, dtype)     # [T,Hv]
    S_all = (np.zeros((N, Hv, V, K), dtype) if state is None
             else np.asarray(state, dtype).copy())
    out = np.zeros((T, Hv, V), dtype)
    rq, rk = Hv // Hq, Hv // Hk
    C = chunk
    tril_strict = np.tril(np.ones((C, C), bool), -1)
    tril_incl = np.tril(np.ones((C, C), bool), 0)
    for n, (s, e) in enumerate(bounds):
        if e - s <= 0:
            continue                                      # :61-66
        S = S_all[n].copy()                               # [Hv,V,K]
        for cs in range(s, e, C):
            clen = min(C, e - cs)
            Qc = np.zeros((Hv, C, K), dtype); Kc = np.zeros((Hv, C, K), dtype)
            Vc = np.zeros((Hv, C, V), dtype)
            Qc[:, :clen] = np.moveaxis(np.repeat(q[cs:cs + clen], rq, axis=1), 0, 1)
            Kc[:, :clen] = np.moveaxis(np.repeat(k[cs:cs + clen], rk, axis=1), 0, 1)
            Vc[:, :clen] = np.moveaxis(v[cs:cs + clen], 0, 1)
            gam = np.zeros((Hv, C), dtype); bet = np.zeros((Hv, C), dtype)
            gam[:, :clen] = lg[cs:cs + clen].T
            bet[:, :clen] = beta[cs:cs + clen].T
            gam = np.cumsum(gam, axis=1)
            eg = np.exp(gam)
            Gam = np.exp(np.where(tril_incl, gam[:, :, None] - gam[:, None, :], 0.0))
            KK = Kc @ np.swapaxes(Kc, 1, 2)
            A = np.where(tril_strict, -bet[:, :, None] * KK * Gam, 0.0)
            Tt = _tri_inverse_unit_lower(-A)
            P = np.where(tril_incl, (Qc @ np.swapaxes(Kc, 1, 2)) * Gam, 0.0)
            W = Tt @ (Kc * (bet * eg)[:, :, None])
            inter = (Qc * eg[:, :, None]) @ np.swapaxes(S, 1, 2)
            corr = W @ np.swapaxes(S, 1, 2)
            v_new = Tt @ (bet[:, :, None] * Vc) - corr
            o = scale * (inter + P @ v_new)
            out[cs:cs + clen] = np.moveaxis(o[:, :clen], 0, 1)
            g_last = gam[:, clen - 1]
            Kdec = Kc * np.exp(g_last[:, None] - gam)[:, :, None]
            S = S * np.exp(g_last)[:, None, None] + np.swapaxes(v_new, 1, 2) @ Kdec
        S_all[n] = S
    return out, S_all
