"""CPU tests of the C ABI: the library loads, exports every symbol the header
declares, and validates arguments before any device call (these run without a
GPU; no compute entry point is called with valid arguments here)."""
import os
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from gdn_kernel_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))

OK, INVALID, UNSUPPORTED = _lib.GDN_OK, _lib.GDN_ERR_INVALID_ARGUMENT, _lib.GDN_ERR_UNSUPPORTED
FAKE = 0x10000  # non-null, never dereferenced by the *_check functions


def header_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(gdn_[a-z_0-9]+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_library_exports_every_header_symbol(lib):
    names = header_functions()
    assert {"gdn_decode", "gdn_decode_pooled", "gdn_prefill", "gdn_last_error"} <= set(names)
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature in _lib.SIGNATURES"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (gdn_\w+)", out))
    assert set(names) <= exported
    assert exported <= set(names), f"undeclared exports: {exported - set(names)}"


def test_version(lib):
    assert lib.gdn_version() >= 100


def dec_args(**kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, state=FAKE, A_log=FAKE, a=FAKE, dt_bias=FAKE, b=FAKE,
             scale=0.0, output=FAKE, new_state=FAKE + (1 << 30), B=64, Hq=16, Hk=16, Hv=32,
             dk=128, dv=128)
    a.update(kw)
    return [a[k] for k in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "scale",
                           "output", "new_state", "B", "Hq", "Hk", "Hv", "dk", "dv")]


def test_decode_check_accepts_valid(lib):
    assert lib.gdn_decode_check(*dec_args()) == OK
    assert lib.gdn_decode_check(*dec_args(state=None)) == OK            # zero initial state
    assert lib.gdn_decode_check(*dec_args(new_state=FAKE)) == OK        # exact in-place alias
    assert lib.gdn_decode_check(*dec_args(B=0, q=None)) == OK           # empty batch
    assert lib.gdn_decode_check(*dec_args(Hq=4, Hk=8, Hv=32)) == OK     # distinct q/k ratios


@pytest.mark.parametrize("kw,code,frag", [
    (dict(B=-1), INVALID, "batch"),
    (dict(Hv=30), INVALID, "multiple"),
    (dict(Hq=0), INVALID, "positive"),
    (dict(dk=64), UNSUPPORTED, "128"),
    (dict(dv=256), UNSUPPORTED, "128"),
    (dict(q=None), INVALID, "null"),
    (dict(new_state=None), INVALID, "null"),
    (dict(scale=float("nan")), INVALID, "scale"),
    (dict(new_state=FAKE + 4096), INVALID, "overlap"),
])
def test_decode_rejects(lib, kw, code, frag):
    assert lib.gdn_decode_check(*dec_args(**kw)) == code
    assert frag in _lib.last_error()
    # the launching entry point reports the same error without touching a device
    assert lib.gdn_decode(*dec_args(**kw), None) == code


def pool_args(**kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, pool=FAKE, slots=1024, idx=FAKE, A_log=FAKE, a=FAKE,
             dt_bias=FAKE, b=FAKE, scale=0.0, output=FAKE, B=512, Hq=16, Hk=16, Hv=32, dk=128,
             dv=128)
    a.update(kw)
    return [a[k] for k in ("q", "k", "v", "pool", "slots", "idx", "A_log", "a", "dt_bias", "b",
                           "scale", "output", "B", "Hq", "Hk", "Hv", "dk", "dv")]


def test_pooled_check(lib):
    assert lib.gdn_decode_pooled_check(*pool_args()) == OK
    assert lib.gdn_decode_pooled_check(*pool_args(slots=0)) == INVALID
    assert "pool_slots" in _lib.last_error()
    assert lib.gdn_decode_pooled_check(*pool_args(idx=None)) == INVALID
    assert lib.gdn_decode_pooled_check(*pool_args(pool=None)) == INVALID
    assert lib.gdn_decode_pooled(*pool_args(Hv=7), None) == INVALID


def pre_args(**kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, state=FAKE, A_log=FAKE, a=FAKE, dt_bias=FAKE, b=FAKE,
             cu=FAKE, cu_dtype=_lib.GDN_INDEX_INT32, N=32, T=32768, scale=0.0, output=FAKE,
             new_state=FAKE + (1 << 30), Hq=16, Hk=16, Hv=32, dk=128, dv=128)
    a.update(kw)
    return [a[k] for k in ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu",
                           "cu_dtype", "N", "T", "scale", "output", "new_state", "Hq", "Hk", "Hv",
                           "dk", "dv")]


def test_header_constants_match_the_python_binding():
    """Every integer #define of include/gdn_kernel_amd.h (a literal, or a literal shifted
    left) has the same value in _lib."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    text = open(os.path.join(root, "include", "gdn_kernel_amd.h")).read()
    defs = dict(re.findall(r"^#define (GDN_[A-Z0-9_]+) \(?([0-9LL <]+?)\)?\s*(?:/\*.*)?$", text, re.M))
    assert {"GDN_OK", "GDN_ERR_UNSUPPORTED", "GDN_INDEX_INT64", "GDN_MAX_HEADS",
            "GDN_PREFILL_NO_ALLOC_SCRATCH_BYTES", "GDN_PREFILL_DROPIN_SCRATCH_BYTES",
            "GDN_PREFILL_DROPIN_TWO_KERNEL_TOKENS"} <= set(defs)
    for name, value in defs.items():
        parts = [int(x.strip().rstrip("L")) for x in value.split("<<")]
        expected = parts[0] << parts[1] if len(parts) == 2 else parts[0]
        assert getattr(_lib, name) == expected, name


def test_head_count_limit(lib):
    """Head counts up to GDN_MAX_HEADS (65,536) pass validation; above it both entry
    points refuse with GDN_ERR_UNSUPPORTED before any device call (the kernels' per-chunk
    row offsets are 32-bit)."""
    limit = 65536
    far = FAKE + (1 << 44)   # new_state well clear of the (huge) state range
    assert lib.gdn_prefill_check(*pre_args(N=1, T=64, Hq=1, Hk=1, Hv=limit, new_state=far)) == OK
    assert lib.gdn_decode_check(*dec_args(B=1, Hq=1, Hk=1, Hv=limit, new_state=far)) == OK
    assert lib.gdn_prefill_check(*pre_args(N=1, T=64, Hq=1, Hk=1, Hv=2 * limit, new_state=far)) == UNSUPPORTED
    assert "num_v_heads" in _lib.last_error()
    assert lib.gdn_decode_check(*dec_args(B=1, Hq=1, Hk=1, Hv=2 * limit, new_state=far)) == UNSUPPORTED
    assert "num_v_heads" in _lib.last_error()


def test_prefill_check_accepts_valid(lib):
    assert lib.gdn_prefill_check(*pre_args()) == OK
    assert lib.gdn_prefill_check(*pre_args(cu_dtype=_lib.GDN_INDEX_INT64)) == OK
    assert lib.gdn_prefill_check(*pre_args(state=None)) == OK
    assert lib.gdn_prefill_check(*pre_args(N=0, cu=None)) == OK
    assert lib.gdn_prefill_check(*pre_args(T=0, q=None, k=None, v=None, a=None, b=None,
                                           output=None)) == OK          # only empty sequences


@pytest.mark.parametrize("kw,code,frag", [
    (dict(cu_dtype=2), INVALID, "cu_seqlens_dtype"),
    (dict(N=-1), INVALID, "num_seqs"),
    (dict(T=-5), INVALID, "total_tokens"),
    (dict(cu=None), INVALID, "null"),
    (dict(Hk=3), INVALID, "multiple"),
    (dict(dk=96), UNSUPPORTED, "128"),
    (dict(new_state=FAKE + 64), INVALID, "overlap"),
])
def test_prefill_rejects(lib, kw, code, frag):
    assert lib.gdn_prefill_check(*pre_args(**kw)) == code
    assert frag in _lib.last_error()
    assert lib.gdn_prefill(*pre_args(**kw), None) == code


@pytest.mark.parametrize("kw,code,frag", [
    (dict(N=-1), INVALID, "num_seqs"),
    (dict(dk=96), UNSUPPORTED, "128"),
])
def test_prefill_fault_injection_rejects(lib, kw, code, frag):
    """The testing entry point validates like gdn_prefill, and its hooks must be >= 0;
    every case fails before any device call."""
    assert lib.gdn_prefill_fault_injection(*pre_args(**kw), 0, 0, None, None) == code
    assert frag in _lib.last_error()
    for spin, ready in ((-1, 0), (0, -2)):
        assert lib.gdn_prefill_fault_injection(*pre_args(), spin, ready, None, None) == INVALID
        assert "spin_limit" in _lib.last_error()


def test_prefill_workspace_size(lib):
    """Bytes of the two-kernel prefill path: N ceil(T / 64) Hv chunk images of 19,200
    bytes (of T~ hi, T~ lo and P each the operand rows the state pass reads: 32 rows of
    32 and 32 rows of 64 bf16; then three 64-float gate vectors) for batches whose chains
    are split 4 or 8 ways across workgroups (at most 64 chains on 256 CUs), 0 otherwise.
    Without a GPU the CU count defaults to 256."""
    image = 3 * (32 * 32 + 32 * 64) * 2 + 3 * 64 * 4
    assert image == 19200
    assert lib.gdn_prefill_workspace_size(1, 4096, 32) == 64 * 32 * image
    assert lib.gdn_prefill_workspace_size(3, 100, 8) == 3 * 2 * 8 * image
    assert lib.gdn_prefill_workspace_size(2, 4096, 32) == 2 * 64 * 32 * image    # 64 chains
    assert lib.gdn_prefill_workspace_size(3, 4096, 32) == 0                      # 96 chains: one kernel
    assert lib.gdn_prefill_workspace_size(5, 4096, 32) == 0
    for n, t, hv in ((0, 100, 8), (1, 0, 8), (1, 100, 0), (-1, 100, 8), (1, -5, 8)):
        assert lib.gdn_prefill_workspace_size(n, t, hv) == 0
    assert lib.gdn_prefill_workspace_size(1, 1 << 24, 32) == 0                   # above the 2 GiB cap


def test_prefill_with_workspace_validates(lib):
    """gdn_prefill_with_workspace validates like gdn_prefill, then rejects a workspace
    below the reported size or not 16-byte aligned; every case fails before any device
    call."""
    small = pre_args(N=1, T=4096)
    need = lib.gdn_prefill_workspace_size(1, 4096, 32)
    assert lib.gdn_prefill_with_workspace(*pre_args(N=-1), FAKE, need, None) == INVALID
    assert "num_seqs" in _lib.last_error()
    assert lib.gdn_prefill_with_workspace(*pre_args(dk=96), FAKE, need, None) == UNSUPPORTED
    assert lib.gdn_prefill_with_workspace(*small, FAKE, need - 1, None) == INVALID
    assert "workspace_bytes" in _lib.last_error()
    assert lib.gdn_prefill_with_workspace(*small, FAKE + 8, need, None) == INVALID
    assert "aligned" in _lib.last_error()


def test_decode_variant_entry_points_validate(lib):
    """The launch-shape testing entry points reject out-of-range shapes (and whatever
    gdn_decode rejects) before any device call."""
    n = lib.gdn_decode_num_variants()
    assert n == 16
    for bad in (-1, n):
        assert lib.gdn_decode_with_variant(*dec_args(), bad, None) == INVALID
        assert "variant" in _lib.last_error()
        assert lib.gdn_decode_pooled_with_variant(*pool_args(), bad, None) == INVALID
    assert lib.gdn_decode_with_variant(*dec_args(dk=64), 0, None) == UNSUPPORTED
    assert lib.gdn_decode_pooled_with_variant(*pool_args(slots=0), 0, None) == INVALID


def test_last_error_is_cleared_on_success(lib):
    lib.gdn_decode_check(*dec_args(B=-1))
    assert _lib.last_error()
    assert lib.gdn_decode_check(*dec_args()) == OK
    assert _lib.last_error() == ""


def test_check_maps_codes_to_exceptions():
    _lib.load().gdn_decode_check(*dec_args(dk=64))
    with pytest.raises(ValueError, match="128"):
        _lib.check(UNSUPPORTED)
    with pytest.raises(_lib.GDNError):
        _lib.check(_lib.GDN_ERR_DEVICE)


def test_launch_size_is_bounded_in_work_items(lib):
    """A launch's grid times its workgroup size must fit in 32 bits.  Decode takes 1024
    work-items per (batch row, v-head) in its default launch shape (8 rows per
    wavefront), so B * Hv may reach 4,194,303; shapes with 2 rows per wavefront take
    4096 (B * Hv up to 1,048,575).  Prefill's one-kernel launch takes 512 per (sequence,
    v-head) chain, so N * Hv may reach 8,388,607.  Larger requests are rejected before
    any device call instead of failing at launch."""
    assert lib.gdn_decode_check(*dec_args(B=131071, state=None)) == OK          # 4,194,272 heads
    assert lib.gdn_decode_check(*dec_args(B=131072, state=None)) == INVALID     # 4,194,304
    assert "work-items" in _lib.last_error()
    assert lib.gdn_decode(*dec_args(B=131072, state=None), None) == INVALID
    assert lib.gdn_decode_pooled_check(*pool_args(B=131071)) == OK
    assert lib.gdn_decode_pooled_check(*pool_args(B=131072)) == INVALID
    assert lib.gdn_decode_pooled(*pool_args(B=131072), None) == INVALID
    # variant 15: 2 rows per wavefront, one wavefront per workgroup
    assert lib.gdn_decode_with_variant(*dec_args(B=32768, state=None), 15, None) == INVALID
    assert "work-items" in _lib.last_error()
    assert lib.gdn_decode_pooled_with_variant(*pool_args(B=32768), 15, None) == INVALID
    assert lib.gdn_prefill_check(*pre_args(N=262143, state=None)) == OK           # 8,388,576 chains
    assert lib.gdn_prefill_check(*pre_args(N=262144, state=None)) == INVALID      # 8,388,608
    assert "work-items" in _lib.last_error()
    assert lib.gdn_prefill(*pre_args(N=262144, state=None), None) == INVALID


def test_prefill_giveups_reporting(lib):
    """gdn_prefill_giveups (the device count of prefill hand-off waits that gave up)
    rejects a null destination before any device call; without a usable GPU it reports
    a device error with a message instead of a count, and the Python helper raises."""
    assert lib.gdn_prefill_giveups(None, 0) == INVALID
    assert "count" in _lib.last_error()
    count = ctypes.c_uint64(12345)
    rc = lib.gdn_prefill_giveups(ctypes.byref(count), 0)
    assert rc in (OK, _lib.GDN_ERR_DEVICE)
    if rc == OK:
        assert count.value < 12345
    else:
        assert "gdn_prefill_giveups" in _lib.last_error()
        assert count.value == 12345


def test_decode_pool_conflicts_reporting(lib):
    """gdn_decode_pool_conflicts (the device count of pooled decode rows skipped because
    another row named their slot) rejects a null destination before any device call;
    without a usable GPU it reports a device error and leaves the destination alone."""
    assert lib.gdn_decode_pool_conflicts(None, 1) == INVALID
    assert "count" in _lib.last_error()
    count = ctypes.c_uint64(777)
    rc = lib.gdn_decode_pool_conflicts(ctypes.byref(count), 0)
    assert rc in (OK, _lib.GDN_ERR_DEVICE)
    if rc != OK:
        assert "gdn_decode_pool_conflicts" in _lib.last_error()
        assert count.value == 777


def test_static_device_bytes_match_the_header(lib):
    """gdn_static_device_bytes (device memory the library holds on every device it is
    loaded onto) is the two prefill scratch arrays the header names plus 12 bytes of
    device counters (prefill give-ups, 4; pooled-decode conflicts, 8): 192 MiB."""
    want = _lib.GDN_PREFILL_DROPIN_SCRATCH_BYTES + _lib.GDN_PREFILL_NO_ALLOC_SCRATCH_BYTES + 12
    assert lib.gdn_static_device_bytes() == want
    assert _lib.GDN_PREFILL_DROPIN_SCRATCH_BYTES == 128 << 20
    assert _lib.GDN_PREFILL_NO_ALLOC_SCRATCH_BYTES == 64 << 20
    assert want == (192 << 20) + 12
    # the drop-in array holds config 3's images (one 4,096-token sequence, 32 v-heads)
    # and those of one sequence of up to 13,952 tokens
    assert lib.gdn_prefill_workspace_size(1, 4096, 32) <= _lib.GDN_PREFILL_DROPIN_SCRATCH_BYTES
    assert lib.gdn_prefill_workspace_size(1, 13952, 32) <= _lib.GDN_PREFILL_DROPIN_SCRATCH_BYTES
    assert lib.gdn_prefill_workspace_size(1, 13953, 32) > _lib.GDN_PREFILL_DROPIN_SCRATCH_BYTES
