"""The TVM-FFI shims (gdn_kernel_amd/csrc/tvm_ffi): without tvm-ffi (as in this image)
the build skips them; their exported `kernel` keeps the reference's signatures
(kernel.cu:101-113, kernel_prefill.cu:300-306) and calls only C-ABI functions the
header declares, with as many arguments as the declaration has."""
import re
from pathlib import Path

import pytest

from gdn_kernel_amd import build as b

ROOT = Path(__file__).resolve().parents[1]
HEADER = (ROOT / "include" / "gdn_kernel_amd.h").read_text()

REFERENCE_PARAMS = {
    "decode": ("GDNDecodeKernel", ["q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "scale",
                                   "output", "new_state"]),
    "prefill": ("GDNPrefillKernel", ["q", "k", "v", "state", "A_log", "a", "dt_bias", "b",
                                     "cu_seqlens", "scale", "output", "new_state"]),
}


def _strip_comments(text):
    return re.sub(r"//[^\n]*", "", re.sub(r"/\*.*?\*/", "", text, flags=re.S))


def _declared_arity(name):
    m = re.search(r"\b" + name + r"\s*\(([^;]*?)\)\s*;", _strip_comments(HEADER), re.S)
    assert m, f"{name} is not declared in the header"
    return len([x for x in m.group(1).split(",") if x.strip() and x.strip() != "void"])


def _call_arity(text, name):
    i = text.index(name + "(") + len(name) + 1
    depth, args = 1, 0
    while depth:
        c = text[i]
        if c in "([{":
            depth += 1
        elif c in ")]}":
            depth -= 1
        elif c == "," and depth == 1:
            args += 1
        i += 1
    return args + 1


def test_build_skips_without_tvm_ffi(monkeypatch):
    monkeypatch.delenv("TVM_FFI_INCLUDE", raising=False)
    try:
        import tvm_ffi  # noqa: F401
        pytest.skip("tvm-ffi is installed here")
    except ImportError:
        pass
    assert b.tvm_ffi_paths() is None
    assert b.build_tvm_ffi() == {}
    monkeypatch.setenv("TVM_FFI_INCLUDE", str(ROOT / "nonexistent"))
    assert b.tvm_ffi_paths() is None


@pytest.mark.parametrize("op", ["decode", "prefill"])
def test_shim_signature_and_calls(op):
    src = _strip_comments((b.CSRC / b.TVM_FFI_SHIMS[op]).read_text())
    fn, params = REFERENCE_PARAMS[op]
    assert re.search(r"TVM_FFI_DLL_EXPORT_TYPED_FUNC\(\s*kernel\s*,\s*" + fn + r"\s*\)", src)
    m = re.search(r"void " + fn + r"\((.*?)\)\s*\{", src, re.S)
    names = [re.split(r"\s+", x.strip())[-1] for x in m.group(1).split(",")]
    assert names == params
    called = set(re.findall(r"\b(gdn_[a-z_0-9]+)\s*\(", src))
    assert called == {f"gdn_{op}", "gdn_last_error"}
    assert _call_arity(src, f"gdn_{op}") == _declared_arity(f"gdn_{op}")


EXPECTED_DTYPES = {
    "decode": {"q": "kBF16", "k": "kBF16", "v": "kBF16", "state": "kF32", "A_log": "kF32",
               "a": "kBF16", "dt_bias": "kF32", "b": "kBF16", "output": "kBF16", "new_state": "kF32"},
    "prefill": {"q": "kBF16", "k": "kBF16", "v": "kBF16", "state": "kF32", "A_log": "kF32",
                "a": "kBF16", "dt_bias": "kF32", "b": "kBF16", "cu_seqlens": "kIndex",
                "output": "kBF16", "new_state": "kF32"},
}


@pytest.mark.parametrize("op", ["decode", "prefill"])
def test_shim_checks_every_tensor(op):
    """Before the C-ABI call each shim checks every tensor argument (check_tensor: dtype,
    rank, extents, device, contiguity) with the dtype the binding requires, the
    optional state only when it is not a null tensor, as binding.py does."""
    src = _strip_comments((b.CSRC / b.TVM_FFI_SHIMS[op]).read_text())
    calls = dict(re.findall(r'check_tensor\(\s*(\w+)\s*,\s*"\1"\s*,\s*DType::(\w+)', src))
    assert calls == EXPECTED_DTYPES[op]
    assert re.search(r"if\s*\(\s*state\.data_ptr\(\)\s*!=\s*nullptr\s*\)\s*check_tensor\(\s*state", src)
    assert src.index("check_tensor(new_state") < src.index(f"gdn_{op}(")


def test_check_helper_covers_dtype_rank_device_contiguity():
    src = _strip_comments((b.CSRC / "tvm_ffi" / "check.hpp").read_text())
    body = src[src.index("inline void check_tensor"):]
    for needle in ("dtype_ok(t.dtype()", "t.ndim()", "t.size(i)", "t.device()", "t.stride(j)",
                   "TVM_FFI_THROW(ValueError)"):
        assert needle in body, needle
    assert "kDLBfloat" in src and "kDLFloat" in src and "kDLInt" in src


STUB = ROOT / "tests" / "tvm_ffi_stub"

EXPECTED_RUNS = {
    "decode": {
        "valid_empty_batch": "ok",
        "null_state": "ok",
        "q_dtype": "ValueError: q must be bfloat16",
        "k_rank": "ValueError: q, k, v must be 4-D",
        "output_extent": "ValueError: output dim 3 must be 128 (got 64)",
        "state_device": "ValueError: state is on another device than q",
        "state_strided": "ValueError: state must be contiguous",
        "a_dtype": "ValueError: a must be bfloat16",
        "new_state_shape": "ValueError: new_state dim 3 must be 128 (got 64)",
        "c_abi_head_ratio": "RuntimeError: num_v_heads (4) must be a multiple of num_q_heads (3)",
        "c_abi_head_dim": "RuntimeError: only head_dim_k == head_dim_v == 128",
    },
    "prefill": {
        "valid_no_sequences": "ok",
        "valid_leading_one": "ok",
        "valid_int64_offsets": "ok",
        "cu_dtype": "ValueError: cu_seqlens must be int32 or int64",
        "cu_rank": "ValueError: cu_seqlens must be [N + 1]",
        "rank_mismatch": "ValueError: q, k, v must have the same rank",
        "state_shape": "ValueError: state dim 0 must be 0 (got 1)",
        "output_device": "ValueError: output is on another device than q",
        "b_strided": "ValueError: b must be contiguous",
        "c_abi_head_ratio": "RuntimeError: num_v_heads (4) must be a multiple of num_q_heads (3)",
    },
}


@pytest.mark.parametrize("op", ["decode", "prefill"])
def test_shim_compiles_and_checks_against_stand_in_types(op, tmp_path):
    """Each shim compiled with g++ against tests/tvm_ffi_stub -- a stand-in for the
    tvm-ffi types it uses (TensorView's members, DLPack structs, TVM_FFI_THROW), not
    tvm-ffi itself, which this image lacks -- and linked with the built library, then
    run on host tensors: valid empty batches pass through to the C ABI and return; each
    malformed tensor (dtype, rank, extent, device, strides) raises the shim's ValueError
    before the C ABI; requests the C ABI rejects (head ratio, head dim) raise its
    RuntimeError with gdn_last_error's message.  No case reaches a device call.  This
    pins the shims' logic; their fit to the real tvm-ffi headers stays unverified here."""
    from gdn_kernel_amd import _lib
    import shutil
    import subprocess
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    exe = tmp_path / f"shim_{op}"
    cmd = [gxx, "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{STUB}", f"-I{ROOT / 'include'}",
           f"-I{b.CSRC / 'tvm_ffi'}", str(STUB / "shim_driver.cpp"),
           f"-L{_lib.LIB_PATH.parent}", "-lgdn_kernel_amd", f"-Wl,-rpath,{_lib.LIB_PATH.parent}",
           "-o", str(exe)]
    if op == "decode":
        cmd.insert(1, "-DGDN_SHIM_DECODE")
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    got = dict(line.split(": ", 1) for line in run.stdout.splitlines())
    assert set(got) == set(EXPECTED_RUNS[op])
    for case, want in EXPECTED_RUNS[op].items():
        assert got[case].startswith(want), f"{case}: {got[case]!r}"
