"""Build ``libgdn_kernel_amd.so`` (gfx950) in-tree with hipcc.

Usage: ``python -m gdn_kernel_amd.build`` (or ``build()`` from Python).
The shared library is written next to this file so that it travels with the
source tree; there is no JIT cache and no installation step.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libgdn_kernel_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ["gdn_decode.hip", "gdn_prefill.hip", "gdn_capi.cpp"]
HEADERS = ["gdn_common.hpp", "gdn_launch.hpp"]

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Wno-unused-function",
    # No packed-fp32 VALU ops in device code (v_pk_{add,mul,fma}_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Everything the library's code depends on, relative to the repository root: the
# C headers and the HIP/C++ sources and headers.
BUILD_INPUTS = ["include/gdn_kernel_amd.h", "include/gdn_kernel_amd_testing.h",
                *(f"gdn_kernel_amd/csrc/{f}" for f in SOURCES + HEADERS)]


def source_digest(root: Path | None = None) -> str:
    """Build id of the library: 16 hex digits of SHA-256 over the build inputs under
    ``root`` (default: this tree), each as path, NUL, content, NUL, then the
    compiler flags.  Compiled into the library (gdn_build_id), so a library can be
    matched with the exact sources it was built from."""
    root = Path(root) if root is not None else PKG_DIR.parent
    h = hashlib.sha256()
    for rel in BUILD_INPUTS:
        h.update(rel.encode() + b"\0" + (root / rel).read_bytes() + b"\0")
    h.update(" ".join(HIPCC_FLAGS).encode())
    return h.hexdigest()[:16]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def build(verbose: bool = False, out: Path | None = None) -> Path:
    """Compile every HIP/C++ source of the library into one shared object."""
    out = Path(out) if out else LIB_PATH
    tmp = out.with_suffix(".so.tmp")
    srcs = [str(CSRC / s) for s in SOURCES]
    cmd = [hipcc(), *HIPCC_FLAGS, f'-DGDN_BUILD_ID="{source_digest()}"', "-I",
           str(PKG_DIR.parent / "include"), *srcs, "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass reports the device-only target feature as unknown; drop that noise.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if noise not in ln]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs))
    os.replace(tmp, out)
    return out


# TVM-FFI exports (one `kernel` symbol per module, as the reference's two solutions):
# host-only C++ over the C ABI, built when the tvm-ffi headers can be found.
TVM_FFI_SHIMS = {"decode": "tvm_ffi/kernel.cpp", "prefill": "tvm_ffi/kernel_prefill.cpp"}


def tvm_ffi_paths() -> dict | None:
    """Include directories (and the library, if known) of an installed tvm-ffi:
    TVM_FFI_INCLUDE / DLPACK_INCLUDE / TVM_FFI_LIB from the environment, else the
    ``tvm_ffi`` Python package's libinfo.  None when the headers are not found."""
    inc = os.environ.get("TVM_FFI_INCLUDE")
    dl = os.environ.get("DLPACK_INCLUDE")
    lib = os.environ.get("TVM_FFI_LIB")
    if not inc:
        try:
            from tvm_ffi import libinfo  # type: ignore
            inc = libinfo.find_include_path()
            dl = dl or libinfo.find_dlpack_include_path()
            lib = lib or libinfo.find_libtvm_ffi()
        except Exception:  # not installed, or a layout this build does not know
            return None
    if not inc or not (Path(inc) / "tvm" / "ffi" / "function.h").exists():
        return None
    return {"include": [d for d in (inc, dl) if d], "lib": lib}


def build_tvm_ffi(verbose: bool = False, paths: dict | None = None) -> dict:
    """Compile the TVM-FFI shims into ``libgdn_kernel_amd_tvm_ffi_{decode,prefill}.so``
    (linked against ``libgdn_kernel_amd.so``, which must be built).  Returns
    {op: path}, or {} when tvm-ffi is not available."""
    paths = paths if paths is not None else tvm_ffi_paths()
    if paths is None:
        if verbose:
            print("tvm-ffi headers not found: TVM-FFI shims not built", flush=True)
        return {}
    cxx = os.environ.get("CXX") or shutil.which("g++") or "c++"
    built = {}
    for op, src in TVM_FFI_SHIMS.items():
        out = PKG_DIR / f"libgdn_kernel_amd_tvm_ffi_{op}.so"
        cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-I", str(PKG_DIR.parent / "include")]
        for d in paths["include"]:
            cmd += ["-I", str(d)]
        cmd += [str(CSRC / src), "-L", str(PKG_DIR), "-lgdn_kernel_amd", "-Wl,-rpath,$ORIGIN"]
        if paths.get("lib"):
            cmd += [str(paths["lib"])]
        cmd += ["-o", str(out)]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"TVM-FFI shim ({op}) failed to build:\n{res.stdout}{res.stderr}")
        built[op] = out
    return built


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(f"built {path}")
    for op, p in build_tvm_ffi(verbose=True).items():
        print(f"built {p} (TVM-FFI `kernel`, {op})")
