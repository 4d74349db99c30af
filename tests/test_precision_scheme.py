"""CPU emulation of the prefill kernel's operand precision scheme.

The HIP prefill kernel runs its chunk products on bf16 MFMA.  q/k/v are exact
bf16 operands; every fp32 operand on the state path (S in X = K S^T, T~ and Y
in v_new = T~ Y, U = d*v_new in the state update, N into the triangular solve)
is split into a bf16 hi + lo pair, and only the output-only products (Q S^T and
P v_new) use a single bf16 operand.  These tests emulate that algorithm in
float64 with each operand rounded the way the kernel feeds it, on inputs with
slow decay (so the state path dominates), and check:

* the kernel's scheme stays inside the state tolerance (rtol 1e-3, atol 1e-5)
  with margin, and the output tolerance (1e-2);
* giving any one state-path operand a single bf16 or fp16 rounding instead of
  the hi/lo pair breaks the state tolerance -- the hi/lo passes (and their VALU
  splitting work) are required, not a safety margin.
"""
import numpy as np
import pytest

from gdn_kernel_amd import workloads
from gdn_kernel_amd.workloads import Heads, to_numpy
from oracle import gdn_oracle as O

C = 64


def _bf16(x):
    return O.bf16_round(x).astype(np.float64)


def _f16(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def _hilo(x):
    """bf16 hi + bf16 lo (the kernel's split of an fp32 operand)."""
    h = _bf16(x)
    return h + _bf16(np.asarray(x, np.float64) - h)


ROUND = {"hilo": _hilo, "bf16": _bf16, "f16": _f16}

# The kernel's scheme (gdn_prefill.hip): state-path operands hi/lo, output-only bf16.
KERNEL = dict(S="hilo", T="hilo", Y="hilo", U="hilo", N="hilo", Sq="bf16", Vn_o="bf16", P="bf16")


def emulate(p, scheme):
    """The kernel's per-chunk algorithm (X = K S^T first, Y = beta (V - e^gamma X),
    v_new = T~ Y, o = scale (e^gamma Q S^T + P v_new), S = e^{gamma_last} S +
    K^T (d v_new)), with operand roundings from ``scheme``."""
    r = lambda key, x: ROUND[scheme[key]](x)
    q, k, v = (to_numpy(p[n]).astype(np.float64) for n in ("q", "k", "v"))
    lg, beta = O.log_gates(to_numpy(p["A_log"]), to_numpy(p["a"]), to_numpy(p["dt_bias"]),
                           to_numpy(p["b"]), np.float64)
    S_all = to_numpy(p["state"]).astype(np.float64).copy()
    cu = p["cu_seqlens"].numpy()
    scale = p["scale"]
    T, Hq, D = q.shape
    Hv = v.shape[1]
    out = np.zeros((T, Hv, D))
    rq = Hv // Hq
    tri_s = np.tril(np.ones((C, C), bool), -1)
    tri_i = np.tril(np.ones((C, C), bool))
    for n in range(len(cu) - 1):
        s, e = int(cu[n]), int(cu[n + 1])
        S = S_all[n].copy()
        for cs in range(s, e, C):
            cl = min(C, e - cs)
            Qc, Kc, Vc = (np.zeros((Hv, C, D)) for _ in range(3))
            Qc[:, :cl] = np.moveaxis(np.repeat(q[cs:cs + cl], rq, 1), 0, 1)
            Kc[:, :cl] = np.moveaxis(np.repeat(k[cs:cs + cl], rq, 1), 0, 1)
            Vc[:, :cl] = np.moveaxis(v[cs:cs + cl], 0, 1)
            gam, bet = np.zeros((Hv, C)), np.zeros((Hv, C))
            gam[:, :cl] = lg[cs:cs + cl].T
            bet[:, :cl] = beta[cs:cs + cl].T
            gam = np.cumsum(gam, 1)
            eg = np.exp(gam)
            Gam = np.exp(np.where(tri_i, gam[:, :, None] - gam[:, None, :], 0.0))
            N = np.where(tri_s, bet[:, :, None] * (Kc @ Kc.swapaxes(1, 2)) * Gam, 0.0)
            Tt = r("T", O._tri_inverse_unit_lower(r("N", N)))
            P = r("P", np.where(tri_i, (Qc @ Kc.swapaxes(1, 2)) * Gam * scale, 0.0))
            X = Kc @ r("S", S).swapaxes(1, 2)
            Xq = Qc @ r("Sq", S).swapaxes(1, 2)
            Vn = Tt @ r("Y", bet[:, :, None] * (Vc - eg[:, :, None] * X))
            o = scale * eg[:, :, None] * Xq + P @ r("Vn_o", Vn)
            out[cs:cs + cl] = np.moveaxis(o[:, :cl], 0, 1)
            U = r("U", np.exp(gam[:, cl - 1:cl] - gam)[:, :, None] * Vn)
            S = S * np.exp(gam[:, cl - 1])[:, None, None] + U.swapaxes(1, 2) @ Kc
        S_all[n] = S
    return O.bf16_round(out), S_all


@pytest.fixture(scope="module")
def case():
    p = workloads.prefill_inputs([400, 130], Heads(2, 2, 4), seed=3, gate="slow", state_scale=0.5)
    args = [to_numpy(p[n]) for n in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b")]
    o_ref, s_ref = O.prefill_chunked(*args, p["cu_seqlens"].numpy(), p["scale"])
    return p, o_ref, s_ref


def _ratios(p, o_ref, s_ref, scheme):
    o, s = emulate(p, scheme)
    rs = np.abs(s - s_ref) / (1e-5 + 1e-3 * np.abs(s_ref))
    ro = np.abs(o - o_ref) / (1e-2 + 1e-2 * np.abs(o_ref))
    return rs.max(), ro.max()


def test_kernel_scheme_meets_tolerances_with_margin(case):
    p, o_ref, s_ref = case
    rs, ro = _ratios(p, o_ref, s_ref, KERNEL)
    assert rs < 0.5, f"state error at {rs:.2f} of the tolerance"
    assert ro < 0.5, f"output error at {ro:.2f} of the tolerance"


@pytest.mark.parametrize("operand", ["S", "T", "Y", "U", "N"])
@pytest.mark.parametrize("single", ["bf16", "f16"])
def test_single_rounding_of_a_state_operand_fails(case, operand, single):
    p, o_ref, s_ref = case
    rs, _ = _ratios(p, o_ref, s_ref, dict(KERNEL, **{operand: single}))
    assert rs > 1.0, (f"{operand} as a single {single} operand kept the state within "
                      f"tolerance ({rs:.2f}); the hi/lo split would be unnecessary")
