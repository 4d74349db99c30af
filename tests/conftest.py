import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")
    config.addinivalue_line("markers", "giveups_expected: a GPU test that makes prefill hand-off "
                                       "waits give up on purpose (through the testing hooks)")
    config.addinivalue_line("markers", "conflicts_expected: a GPU test that gives pooled decode "
                                       "rows sharing a slot on purpose and checks the count")


@pytest.fixture(autouse=True)
def _no_prefill_giveups(request):
    """Around every GPU test: no prefill hand-off wait may give up (the device counter
    that gdn_prefill_giveups reads stays at 0), except in tests that force give-ups
    through the testing hooks and check the count themselves; and no pooled decode row
    is skipped as a slot conflict, except in tests that name a slot twice on purpose."""
    if request.node.get_closest_marker("gpu") is None or \
            request.node.get_closest_marker("giveups_expected") is not None:
        yield
        return
    from gdn_kernel_amd import binding
    binding.prefill_giveups(reset=True)
    check_conflicts = request.node.get_closest_marker("conflicts_expected") is None
    if check_conflicts:
        binding.decode_pool_conflicts(reset=True)
    yield
    assert binding.prefill_giveups() == 0, "a prefill hand-off wait gave up during this test"
    if check_conflicts:
        assert binding.decode_pool_conflicts() == 0, "a pooled decode row was skipped as a conflict"


@pytest.fixture(scope="session")
def gpu():
    """GPU tests never skip silently: without a visible GPU they fail."""
    import torch
    assert torch.cuda.is_available(), "GPU test run without a visible ROCm GPU"
    from gdn_kernel_amd import _lib
    _lib.load()
    return torch.device("cuda:0")


def close_report(got, ref, rtol, atol):
    """(ok, message) for |got - ref| <= atol + rtol*|ref| elementwise."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = ~(err <= bound)
    if not bad.any():
        return True, ""
    i = np.unravel_index(np.argmax(err - bound), err.shape)
    return False, (f"{int(bad.sum())}/{bad.size} elements outside atol={atol} rtol={rtol}; "
                   f"worst at {tuple(int(x) for x in i)}: got {got[i]!r} ref {ref[i]!r}; "
                   f"max abs err {err.max():.3e}")


def assert_close(got, ref, rtol, atol, what=""):
    ok, msg = close_report(got, ref, rtol, atol)
    assert ok, f"{what}: {msg}"
