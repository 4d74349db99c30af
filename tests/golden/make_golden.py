"""Write the small golden fixtures used by the CPU and GPU tests.

The reference ships no golden vectors for this path, so the expected outputs
here come from the float64 oracle (oracle/gdn_oracle.py: the decode definition
of design.md:166-226 and the sequential prefill definition of
prefill_design.md:497-545), whose functions are pinned by tests/test_oracle.py.
These fixtures freeze those outputs so that any later change to the oracle or
to the kernels is measured against the same numbers.

Inputs are stored as bf16 bit patterns (uint16) -- including the fp32 initial
states, whose values are chosen bf16-representable so they store in 2 bytes --
and A_log / dt_bias as float32.  Expected outputs are float32 (pre-rounding
output, final state).  Slow-decay gates are used so that the state path shows in
the outputs.

Run: python -m tests.golden.make_golden
"""
import numpy as np

from oracle import gdn_oracle as O
from tests.golden import path

D = 128


def _bits(x):
    return O.bf16_bits(x)


def _common(r, hv, shape_ab):
    A_log = np.log(r.uniform(0.01, 0.05, hv)).astype(np.float32)
    dt_bias = (0.1 * r.standard_normal(hv)).astype(np.float32)
    a = _bits(r.standard_normal(shape_ab))
    b = _bits(r.standard_normal(shape_ab) - 1.0)
    return A_log, dt_bias, a, b


def unit(x):
    return x / np.linalg.norm(x, axis=-1, keepdims=True)


def make_decode():
    r = np.random.default_rng(20240601)
    B, hq, hv = 2, 1, 2
    q = _bits(unit(r.standard_normal((B, 1, hq, D))))
    k = _bits(unit(r.standard_normal((B, 1, hq, D))))
    v = _bits(r.standard_normal((B, 1, hv, D)))
    A_log, dt_bias, a, b = _common(r, hv, (B, 1, hv))
    state = _bits(0.5 * r.standard_normal((B, hv, D, D)))
    scale = np.float64(1.0 / np.sqrt(D))
    f = O.bits_to_f32
    out, st = O.decode(f(q), f(k), f(v), f(state), A_log, f(a), dt_bias, f(b), scale)
    np.savez_compressed(path("decode_small.npz"), q=q, k=k, v=v, state=state, A_log=A_log,
                        dt_bias=dt_bias, a=a, b=b, scale=scale,
                        out_ref=out.astype(np.float32), state_ref=st.astype(np.float32))


def make_prefill():
    r = np.random.default_rng(20240602)
    lengths = [67, 0, 13]
    T, N, hq, hv = sum(lengths), len(lengths), 1, 2
    q = _bits(unit(r.standard_normal((T, hq, D))))
    k = _bits(unit(r.standard_normal((T, hq, D))))
    v = _bits(r.standard_normal((T, hv, D)))
    A_log, dt_bias, a, b = _common(r, hv, (T, hv))
    state = _bits(0.5 * r.standard_normal((N, hv, D, D)))
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    scale = np.float64(1.0 / np.sqrt(D))
    f = O.bits_to_f32
    out, st = O.prefill_sequential(f(q), f(k), f(v), f(state), A_log, f(a), dt_bias, f(b), cu,
                                   scale)
    np.savez_compressed(path("prefill_small.npz"), q=q, k=k, v=v, state=state, A_log=A_log,
                        dt_bias=dt_bias, a=a, b=b, cu_seqlens=cu, scale=scale,
                        out_ref=out.astype(np.float32), state_ref=st.astype(np.float32))


if __name__ == "__main__":
    make_decode()
    make_prefill()
    print("wrote", path("decode_small.npz"), path("prefill_small.npz"))
