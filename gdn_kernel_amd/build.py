"""Build ``libgdn_kernel_amd.so`` (gfx950) in-tree with hipcc.

Usage: ``python -m gdn_kernel_amd.build`` (or ``build()`` from Python).
The shared library is written next to this file so that it travels with the
source tree; there is no JIT cache and no installation step.
"""
from __future__ import annotations

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
    cmd = [hipcc(), *HIPCC_FLAGS, "-I", str(PKG_DIR.parent / "include"), *srcs, "-o", str(tmp)]
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


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(f"built {path}")
