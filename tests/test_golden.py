"""CPU: the oracle reproduces the committed golden fixtures (all three prefill
forms agree with them too)."""
import numpy as np

from oracle import gdn_oracle as O
from tests.conftest import assert_close
from tests.golden import path

f = O.bits_to_f32


def test_decode_fixture():
    fx = np.load(path("decode_small.npz"))
    out, st = O.decode(f(fx["q"]), f(fx["k"]), f(fx["v"]), f(fx["state"]), fx["A_log"],
                       f(fx["a"]), fx["dt_bias"], f(fx["b"]), float(fx["scale"]))
    assert_close(out, fx["out_ref"], 1e-6, 1e-7, "output")
    assert_close(st, fx["state_ref"], 1e-6, 1e-7, "state")
    assert np.abs(fx["out_ref"]).max() > 0.05       # the state path shows in the output


def test_prefill_fixture_all_forms():
    fx = np.load(path("prefill_small.npz"))
    args = (f(fx["q"]), f(fx["k"]), f(fx["v"]), f(fx["state"]), fx["A_log"], f(fx["a"]),
            fx["dt_bias"], f(fx["b"]), fx["cu_seqlens"], float(fx["scale"]))
    for fn in (O.prefill_sequential, O.prefill_chunked):
        out, st = fn(*args)
        assert_close(out, fx["out_ref"], 1e-6, 1e-7, f"{fn.__name__} output")
        assert_close(st, fx["state_ref"], 1e-6, 1e-7, f"{fn.__name__} state")
    # the empty middle sequence passes its initial state through
    np.testing.assert_array_equal(fx["state_ref"][1], f(fx["state"])[1])
