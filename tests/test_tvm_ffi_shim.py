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
