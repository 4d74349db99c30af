"""Pins the CPU oracle (oracle/gdn_oracle.py) against what the mathematics fixes.

The reference ships no golden vectors or tests for this path, so each oracle
function is checked against closed forms, invariants and independent
restatements (the paper's matrix recurrence, the FLA recurrent and chunk forms,
the reference kernel's per-chunk algorithm) -- chosen so that a plausible
mistake fails at least one check.  The mutant tests plant such mistakes in
wrappers around the oracle and confirms the checks catch them (the
``test_*_catch_*`` tests).
"""
import math

import numpy as np
import pytest
import torch

from oracle import gdn_oracle as O
from tests.conftest import assert_close, close_report

RTOL = 1e-10
ATOL = 1e-12


def bf(x):
    return O.bf16_round(x).astype(np.float64)


def unit(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def decode_case(B=2, Hq=2, Hk=2, Hv=4, K=16, V=16, seed=0, gate="baseline", state_scale=0.05):
    r = np.random.default_rng(seed)
    q = bf(unit(r.standard_normal((B, 1, Hq, K))))
    k = bf(unit(r.standard_normal((B, 1, Hk, K))))
    v = bf(r.standard_normal((B, 1, Hv, V)))
    lo, hi = (1.0, 16.0) if gate == "baseline" else (0.01, 0.05)
    A_log = np.log(r.uniform(lo, hi, Hv))
    dt_bias = 0.1 * r.standard_normal(Hv)
    a = bf(r.standard_normal((B, 1, Hv)))
    b = bf(r.standard_normal((B, 1, Hv)))
    state = state_scale * r.standard_normal((B, Hv, V, K))
    return dict(q=q, k=k, v=v, state=state, A_log=A_log, a=a, dt_bias=dt_bias, b=b, scale=None)


def prefill_case(lengths, Hq=2, Hk=2, Hv=4, K=16, V=16, seed=0, gate="slow", state_scale=0.5,
                 with_state=True):
    r = np.random.default_rng(seed)
    T = int(sum(lengths))
    N = len(lengths)
    q = bf(unit(r.standard_normal((T, Hq, K))))
    k = bf(unit(r.standard_normal((T, Hk, K))))
    v = bf(r.standard_normal((T, Hv, V)))
    lo, hi = (1.0, 16.0) if gate == "baseline" else (0.01, 0.05)
    A_log = np.log(r.uniform(lo, hi, Hv))
    dt_bias = 0.1 * r.standard_normal(Hv)
    a = bf(r.standard_normal((T, Hv)))
    b = bf(r.standard_normal((T, Hv)))
    state = state_scale * r.standard_normal((N, Hv, V, K)) if with_state else None
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    return dict(q=q, k=k, v=v, state=state, A_log=A_log, a=a, dt_bias=dt_bias, b=b,
                cu_seqlens=cu, scale=None)


# --------------------------------------------------------------------------- helpers
def test_bf16_round_known_values():
    one = 1.0
    ulp = 2.0 ** -7
    vals = np.array([one, one + ulp / 2, one + 1.5 * ulp, -3.0, 0.0, 65504.0, 1e-40], np.float32)
    got = O.bf16_round(vals)
    assert got[0] == 1.0
    assert got[1] == 1.0                       # tie -> even
    assert got[2] == one + 2 * ulp             # tie -> even (upwards)
    assert got[3] == -3.0 and got[4] == 0.0
    assert np.isnan(O.bf16_round(np.array([np.nan], np.float32)))[0]


def test_bf16_round_matches_torch():
    r = np.random.default_rng(1)
    x = (r.standard_normal(100000) * np.exp(r.uniform(-30, 30, 100000))).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.bf16_bits(x), ref)


# --------------------------------------------------------------------------- gates
def test_softplus_threshold_and_closed_form():
    xs = np.array([-30.0, -5.0, -1e-3, 0.0, 0.7, 5.0, 19.999, 20.0, 20.001, 50.0])
    got = O.softplus(xs)
    for x, y in zip(xs, got):
        want = x if x > 20 else math.log1p(math.exp(x))
        assert y == pytest.approx(want, rel=1e-14, abs=1e-300)
    # torch's softplus uses the same threshold
    t = torch.nn.functional.softplus(torch.tensor(xs, dtype=torch.float64)).numpy()
    np.testing.assert_allclose(got, t, rtol=1e-14)


def test_gates_closed_form_and_limits():
    r = np.random.default_rng(2)
    A_log = np.log(r.uniform(1, 16, 8))
    dt = 0.1 * r.standard_normal(8)
    a = r.standard_normal((5, 8))
    b = r.standard_normal((5, 8))
    g, beta = O.gates(A_log, a, dt, b)
    for i in range(5):
        for h in range(8):
            x = a[i, h] + dt[h]
            sp = x if x > 20 else math.log1p(math.exp(x))
            assert g[i, h] == pytest.approx(math.exp(-math.exp(A_log[h]) * sp), rel=1e-13)
            assert beta[i, h] == pytest.approx(1 / (1 + math.exp(-b[i, h])), rel=1e-14)
    lg, beta2 = O.log_gates(A_log, a, dt, b)
    np.testing.assert_allclose(np.exp(lg), g, rtol=1e-13)
    np.testing.assert_array_equal(beta2, beta)
    # limits: A_log = -inf -> g = 1; b = +-inf -> beta in {0, 1}
    g, beta = O.gates(np.array([-np.inf]), np.array([[3.0]]), np.array([0.0]),
                      np.array([[np.inf]]))
    assert g[0, 0] == 1.0 and beta[0, 0] == 1.0
    _, beta = O.gates(np.array([0.0]), np.array([[0.0]]), np.array([0.0]), np.array([[-np.inf]]))
    assert beta[0, 0] == 0.0


def test_default_scale():
    assert O.default_scale(None, 128) == 1 / math.sqrt(128)
    assert O.default_scale(0.0, 128) == 1 / math.sqrt(128)
    assert O.default_scale(0.25, 128) == 0.25


# --------------------------------------------------------------------------- decode
def _g_beta(c):
    g, beta = O.gates(c["A_log"], c["a"], c["dt_bias"], c["b"])
    return g[:, 0], beta[:, 0]


def test_decode_zero_state_beta_one():
    """S = 0, beta = 1: S' = v (x) k, o = scale (q.k) v."""
    c = decode_case(Hq=4, Hk=4, Hv=4)
    c["b"] = np.full_like(c["b"], np.inf)
    o, S = O.decode(c["q"], c["k"], c["v"], None, c["A_log"], c["a"], c["dt_bias"], c["b"], 0.3)
    q, k, v = c["q"][:, 0], c["k"][:, 0], c["v"][:, 0]
    assert_close(S, v[..., :, None] * k[..., None, :], RTOL, ATOL, "S'")
    assert_close(o[:, 0], 0.3 * (q * k).sum(-1)[..., None] * v, RTOL, ATOL, "o")


def test_decode_beta_zero_is_pure_decay():
    """beta = 0: S' = g S, o = scale g S q."""
    c = decode_case(Hq=4, Hk=4, Hv=4)
    c["b"] = np.full_like(c["b"], -np.inf)
    o, S = O.decode(**c)
    g, _ = _g_beta(c)
    assert_close(S, g[..., None, None] * c["state"], RTOL, ATOL, "S'")
    want = (g[..., None] * np.einsum("bhvk,bhk->bhv", c["state"], c["q"][:, 0])) / math.sqrt(16)
    assert_close(o[:, 0], want, RTOL, ATOL, "o")


def test_decode_exact_delta_write():
    """g = 1, beta = 1, |k| = 1: the updated state maps k exactly to v."""
    c = decode_case(Hq=4, Hk=4, Hv=4, state_scale=1.0)
    c["A_log"] = np.full_like(c["A_log"], -np.inf)
    c["b"] = np.full_like(c["b"], np.inf)
    k = unit(np.random.default_rng(5).standard_normal(c["k"].shape))   # exactly unit in fp64
    c["k"] = k
    _, S = O.decode(**c)
    assert_close(np.einsum("bhvk,bhk->bhv", S, k[:, 0]), c["v"][:, 0], 1e-12, 1e-12, "S' k")


def test_decode_full_decay():
    """g = 0: S' = beta v (x) k."""
    c = decode_case(Hq=4, Hk=4, Hv=4)
    c["a"] = np.full_like(c["a"], 100.0)       # softplus = 100, exp(A_log) >= 1 -> g = e^-100..
    c["A_log"] = np.full_like(c["A_log"], 10.0)
    _, S = O.decode(**c)
    _, beta = _g_beta(c)
    want = beta[..., None, None] * c["v"][:, 0][..., :, None] * c["k"][:, 0][..., None, :]
    assert_close(S, want, RTOL, ATOL, "S'")


def test_decode_matches_paper_recurrence():
    """S_t = S_{t-1} alpha (I - beta k k^T) + beta v k^T, o = scale S_t q
    (prefill_design.md:67-70, the paper's Eq. 10 in the [V, K] orientation), with
    GQA expansion written out per head."""
    c = decode_case(B=3, Hq=2, Hk=1, Hv=4, K=8, V=12, seed=7, state_scale=1.0)
    o, S = O.decode(**c)
    g, beta = _g_beta(c)
    B, Hv = 3, 4
    for bi in range(B):
        for h in range(Hv):
            q = c["q"][bi, 0, h // 2]
            k = c["k"][bi, 0, h // 4]
            v = c["v"][bi, 0, h]
            S0 = c["state"][bi, h]
            St = g[bi, h] * S0 @ (np.eye(8) - beta[bi, h] * np.outer(k, k)) + beta[bi, h] * np.outer(v, k)
            assert_close(S[bi, h], St, RTOL, ATOL, f"S' b{bi} h{h}")
            assert_close(o[bi, 0, h], St @ q / math.sqrt(8), RTOL, ATOL, f"o b{bi} h{h}")


def test_decode_single_pass_identity():
    """o = scale (g S q + delta (q.k)) with delta = beta (v - g S k) (kernel.cu:59-92)."""
    c = decode_case(seed=3, state_scale=1.0, gate="slow")
    o, _ = O.decode(**c)
    g, beta = _g_beta(c)
    q = np.repeat(c["q"][:, 0], 2, axis=1)
    k = np.repeat(c["k"][:, 0], 2, axis=1)
    gs = g[..., None, None] * c["state"]
    delta = beta[..., None] * (c["v"][:, 0] - np.einsum("bhvk,bhk->bhv", gs, k))
    want = (np.einsum("bhvk,bhk->bhv", gs, q) + delta * (q * k).sum(-1)[..., None]) / 4.0
    assert_close(o[:, 0], want, RTOL, ATOL, "o")


def test_decode_gqa_head_map():
    """v-heads 2j and 2j+1 read qk-head j: same result as a non-GQA call with
    q/k repeated per v-head."""
    c = decode_case(B=2, Hq=2, Hk=2, Hv=4, seed=11)
    o, S = O.decode(**c)
    c2 = dict(c)
    c2["q"] = np.repeat(c["q"], 2, axis=2)
    c2["k"] = np.repeat(c["k"], 2, axis=2)
    o2, S2 = O.decode(**c2)
    np.testing.assert_array_equal(o, o2)
    np.testing.assert_array_equal(S, S2)
    # and the heads really differ: swapping the qk heads changes the result
    c3 = dict(c)
    c3["q"] = c["q"][:, :, ::-1].copy()
    o3, _ = O.decode(**c3)
    assert not np.allclose(o, o3)


def test_decode_null_state_is_zero_state():
    c = decode_case()
    o1, S1 = O.decode(**{**c, "state": None})
    o2, S2 = O.decode(**{**c, "state": np.zeros_like(c["state"])})
    np.testing.assert_array_equal(o1, o2)
    np.testing.assert_array_equal(S1, S2)


def test_decode_float32_close_to_float64():
    c = decode_case(seed=4)
    o64, S64 = O.decode(**c)
    o32, S32 = O.decode(**c, dtype=np.float32)
    assert_close(S32, S64, 1e-5, 1e-7, "S fp32 vs fp64")
    assert_close(o32, o64, 1e-5, 1e-7, "o fp32 vs fp64")


def test_decode_pooled_is_gather_decode_scatter():
    c = decode_case(B=3, seed=9)
    r = np.random.default_rng(9)
    pool = r.standard_normal((6, 4, 16, 16))
    idx = np.array([4, -1, 1])                 # row 1 is padding
    o, new_pool = O.decode_pooled(c["q"], c["k"], c["v"], pool, idx, c["A_log"], c["a"],
                                  c["dt_bias"], c["b"], None)
    sel = [0, 2]
    o_ref, S_ref = O.decode(c["q"][sel], c["k"][sel], c["v"][sel], pool[[4, 1]], c["A_log"],
                            c["a"][sel], c["dt_bias"], c["b"][sel], None)
    np.testing.assert_array_equal(o[sel], o_ref)
    assert not o[1].any()
    np.testing.assert_array_equal(new_pool[[4, 1]], S_ref)
    untouched = [0, 2, 3, 5]
    np.testing.assert_array_equal(new_pool[untouched], pool[untouched])


def test_decode_pooled_conflicting_rows_are_padding():
    """Rows that name a slot another in-range row also names are skipped like padding:
    zero output, the slot keeps its bits; every other row is the plain decode of its
    own slot, computed row by row here."""
    c = decode_case(B=7, seed=12)
    r = np.random.default_rng(12)
    pool = r.standard_normal((8, 4, 16, 16))
    idx = np.array([5, 2, 5, -3, 7, 2, 5])     # slot 5 three times, slot 2 twice, row 3 padding
    conflict = O.pool_conflicts(idx, 8)
    np.testing.assert_array_equal(conflict, [True, True, True, False, False, True, True])
    o, new_pool = O.decode_pooled(c["q"], c["k"], c["v"], pool, idx, c["A_log"], c["a"],
                                  c["dt_bias"], c["b"], None)
    assert not o[[0, 1, 2, 3, 5, 6]].any()
    o4, S4 = O.decode(c["q"][4:5], c["k"][4:5], c["v"][4:5], pool[7:8], c["A_log"], c["a"][4:5],
                      c["dt_bias"], c["b"][4:5], None)
    np.testing.assert_array_equal(o[4:5], o4)
    np.testing.assert_array_equal(new_pool[7], S4[0])
    untouched = [0, 1, 2, 3, 4, 5, 6]
    np.testing.assert_array_equal(new_pool[untouched], pool[untouched])
    assert not O.pool_conflicts(np.array([3, 9, -1, 9]), 8).any()  # out-of-range repeats are padding


# --------------------------------------------------------------------------- prefill
def test_prefill_T1_equals_decode():
    c = prefill_case([1], seed=1, gate="baseline", state_scale=0.05)
    o, S = O.prefill_sequential(**c)
    od, Sd = O.decode(c["q"][:, None], c["k"][:, None], c["v"][:, None], c["state"],
                      c["A_log"], c["a"][:, None], c["dt_bias"], c["b"][:, None], None)
    assert_close(o, od[:, 0], RTOL, ATOL, "o")
    assert_close(S, Sd, RTOL, ATOL, "S")


def test_prefill_equals_chained_decode():
    c = prefill_case([9], seed=2)
    o, S = O.prefill_sequential(**c)
    st = c["state"]
    for t in range(9):
        sl = slice(t, t + 1)
        od, st = O.decode(c["q"][sl][:, None], c["k"][sl][:, None], c["v"][sl][:, None], st,
                          c["A_log"], c["a"][sl][:, None], c["dt_bias"], c["b"][sl][:, None],
                          None)
        assert_close(o[t], od[0, 0], RTOL, ATOL, f"o t={t}")
    assert_close(S, st, RTOL, ATOL, "S")


@pytest.mark.parametrize("C", [16, 32, 64])
@pytest.mark.parametrize("T", [1, 37, 64, 100, 130])
def test_fla_chunk_equals_fla_recurrent(C, T):
    r = np.random.default_rng(T * 100 + C)
    H, K, V = 3, 16, 12
    q = unit(r.standard_normal((T, H, K)))
    k = unit(r.standard_normal((T, H, K)))
    v = r.standard_normal((T, H, V))
    beta = r.uniform(0.05, 0.95, (T, H))
    lg = -r.uniform(0.0, 0.08, (T, H))
    S0 = r.standard_normal((H, K, V))
    o1, S1 = O.recurrent_fla(q, k, v, beta, lg, 0.3, S0)
    o2, S2 = O.chunk_fla(q, k, v, lg, beta, C, 0.3, S0)
    assert_close(o2, o1, 1e-9, 1e-11, "o")
    assert_close(S2, S1, 1e-9, 1e-11, "S")


def test_fla_recurrent_equals_sequential_definition():
    """FLA's log-space, K-major form == the definition's form (after GQA expansion,
    transposing the state to [K, V] and taking log of the gate)."""
    c = prefill_case([50], Hq=4, Hk=4, Hv=4, seed=3)
    o, S = O.prefill_sequential(**c)
    lg, beta = O.log_gates(c["A_log"], c["a"], c["dt_bias"], c["b"])
    S0 = np.swapaxes(c["state"][0], -1, -2)
    o2, S2 = O.recurrent_fla(c["q"], c["k"], c["v"], beta, lg, None, S0)
    assert_close(o2, o, 1e-11, 1e-12, "o")
    assert_close(np.swapaxes(S2, -1, -2), S[0], 1e-11, 1e-12, "S")


@pytest.mark.parametrize("chunk", [16, 64])
@pytest.mark.parametrize("gate", ["baseline", "slow"])
def test_prefill_chunked_equals_sequential(chunk, gate):
    lens = [0, 1, 63, 64, 65, 130, 7, 0]
    c = prefill_case(lens, seed=5, gate=gate)
    o1, S1 = O.prefill_sequential(**c)
    o2, S2 = O.prefill_chunked(**c, chunk=chunk)
    assert_close(o2, o1, 1e-9, 1e-11, "o")
    assert_close(S2, S1, 1e-9, 1e-11, "S")


def test_prefill_beta_zero_is_pure_decay():
    c = prefill_case([40], seed=6)
    c["b"] = np.full_like(c["b"], -np.inf)
    o, S = O.prefill_sequential(**c)
    g, _ = O.gates(c["A_log"], c["a"], c["dt_bias"], c["b"])
    cum = np.cumprod(g, axis=0)                                      # [T, Hv]
    assert_close(S[0], cum[-1][:, None, None] * c["state"][0], RTOL, ATOL, "S_T")
    qe = np.repeat(c["q"], 2, axis=1)
    want = cum[..., None] * np.einsum("hvk,thk->thv", c["state"][0], qe) / 4.0
    assert_close(o, want, RTOL, ATOL, "o")


def test_prefill_varlen_is_independent_sequences():
    lens = [5, 0, 70, 3]
    c = prefill_case(lens, seed=8)
    o, S = O.prefill_sequential(**c)
    cu = c["cu_seqlens"]
    for i, L in enumerate(lens):
        s, e = int(cu[i]), int(cu[i + 1])
        ci = {key: c[key] for key in ("A_log", "dt_bias")}
        oi, Si = O.prefill_sequential(c["q"][s:e], c["k"][s:e], c["v"][s:e], c["state"][i:i + 1],
                                      c["A_log"], c["a"][s:e], c["dt_bias"], c["b"][s:e],
                                      np.array([0, L]), None)
        np.testing.assert_array_equal(o[s:e], oi)
        np.testing.assert_array_equal(S[i], Si[0])
    np.testing.assert_array_equal(S[1], c["state"][1])               # empty sequence


def test_prefill_null_state_is_zero_state():
    c = prefill_case([3, 70], seed=12)
    o1, S1 = O.prefill_sequential(**{**c, "state": None})
    o2, S2 = O.prefill_sequential(**{**c, "state": np.zeros_like(c["state"])})
    np.testing.assert_array_equal(o1, o2)
    np.testing.assert_array_equal(S1, S2)


def test_tri_inverse():
    r = np.random.default_rng(13)
    N = np.tril(r.standard_normal((64, 64)) * 0.2, -1)
    X = O._tri_inverse_unit_lower(N)
    assert_close(X @ (np.eye(64) + N), np.eye(64), 1e-10, 1e-10, "X (I+N)")
    assert np.allclose(np.triu(X, 1), 0) and np.allclose(np.diag(X), 1)


# --------------------------------------------------------------------------- mutants
def _decode_checks(fn):
    """Run a decode implementation through the closed-form checks; return the
    names of the checks it fails."""
    failed = []
    c = decode_case(B=2, Hq=2, Hk=2, Hv=4, K=10, V=10, seed=21, state_scale=1.0, gate="slow")
    o, S = fn(**c)
    g, beta = _g_beta(c)
    for bi in range(2):
        for h in range(4):
            q, k = c["q"][bi, 0, h // 2], c["k"][bi, 0, h // 2]
            v, S0 = c["v"][bi, 0, h], c["state"][bi, h]
            St = g[bi, h] * S0 @ (np.eye(10) - beta[bi, h] * np.outer(k, k)) + beta[bi, h] * np.outer(v, k)
            if not close_report(S[bi, h], St, 1e-9, 1e-12)[0] or \
               not close_report(o[bi, 0, h], St @ q / math.sqrt(10), 1e-9, 1e-12)[0]:
                failed.append("paper_recurrence")
                return failed
    return failed


def _mut_transposed_state(**c):
    st = np.swapaxes(c["state"], -1, -2).copy()
    o, S = O.decode(**{**c, "state": st})
    return o, S


def _mut_wrong_gqa(**c):
    o, S = O.decode(**{**c, "q": c["q"][:, :, ::-1].copy(), "k": c["k"][:, :, ::-1].copy()})
    return o, S


def _mut_no_beta(**c):
    return O.decode(**{**c, "b": np.full_like(c["b"], np.inf)})


def _mut_sign(**c):
    o, S = O.decode(**c)
    g, beta = _g_beta(c)
    gs = g[..., None, None] * c["state"]
    return o, 2 * gs - S                       # S' = gS - k (x) delta  (flipped update)


def _mut_ungated(**c):
    return O.decode(**{**c, "A_log": np.full_like(c["A_log"], -np.inf)})


@pytest.mark.parametrize("mutant", [_mut_transposed_state, _mut_wrong_gqa, _mut_no_beta,
                                    _mut_sign, _mut_ungated])
def test_decode_checks_catch_planted_mistakes(mutant):
    assert _decode_checks(O.decode) == []
    assert _decode_checks(mutant) != [], f"{mutant.__name__} was not caught"


def test_chunk_checks_catch_dropped_inter_decay():
    """A chunked prefill that forgets the e^gamma factor on the inter-chunk term
    fails the chunked == sequential check under slow-decay gates."""
    c = prefill_case([130], seed=14, gate="slow")
    o1, _ = O.prefill_sequential(**c)
    # planted mistake: treat every gate as 1 inside the chunk algorithm only
    bad = dict(c)
    bad["A_log"] = np.full_like(c["A_log"], -np.inf)
    o2, _ = O.prefill_chunked(**bad)
    assert not close_report(o2, o1, 1e-6, 1e-8)[0]


@pytest.mark.parametrize("gate", ["baseline", "slow", "edge"])
def test_torch_definition_matches_oracle_decode(gate):
    """oracle/torch_definition.py (the PyTorch definition of design.md:166-226 that the
    CPU baseline times) computes what the numpy oracle's decode computes: the same fp32
    arithmetic up to summation order, on config-0 heads (16/16/32) and two batch rows."""
    from gdn_kernel_amd import workloads
    from gdn_kernel_amd.workloads import to_numpy
    from oracle.torch_definition import decode_definition
    w = workloads.decode_inputs(2, seed=90, gate=gate, state_scale=0.5)
    o_t, s_t = decode_definition(w["q"], w["k"], w["v"], w["state"], w["A_log"], w["a"],
                                 w["dt_bias"], w["b"], w["scale"])
    o_ref, s_ref = O.decode(*[to_numpy(w[k]) for k in ("q", "k", "v", "state", "A_log", "a",
                                                        "dt_bias", "b")], w["scale"])
    assert o_t.dtype == torch.bfloat16 and s_t.dtype == torch.float32
    assert np.allclose(o_t.double().numpy(), o_ref, rtol=1e-2, atol=1e-2)
    assert np.allclose(s_t.double().numpy(), s_ref, rtol=1e-5, atol=1e-6)
    o0, s0 = decode_definition(w["q"], w["k"], w["v"], None, w["A_log"], w["a"], w["dt_bias"],
                               w["b"], 0.0)
    z = O.decode(*[to_numpy(w[k]) for k in ("q", "k", "v")], None,
                 *[to_numpy(w[k]) for k in ("A_log", "a", "dt_bias", "b")], None)
    assert np.allclose(s0.double().numpy(), z[1], rtol=1e-5, atol=1e-6)
