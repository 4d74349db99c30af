"""Solution packaging (gdn_kernel_amd.pack): config parsing, the solution.json shape,
an exact extract round trip, and that an extracted tree builds and exports the C ABI."""
import ctypes
import json
import re
import subprocess
import sys
from pathlib import Path

import pytest

from gdn_kernel_amd import pack

ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.parametrize("op", ["decode", "prefill"])
def test_pack_solution_shape(op, tmp_path):
    out = tmp_path / "solution.json"
    sol = pack.pack_solution(pack.CONFIG_DIR / f"{op}.toml", ROOT, out)
    on_disk = json.loads(out.read_text())
    assert on_disk == sol
    assert sol["definition"] == f"gdn_{op}_qk16_v32_d128_k_last"
    spec = sol["spec"]
    assert spec["language"] == "hip" and spec["target_hardware"] == ["rocm:gfx950"]
    assert spec["entry_point"] == f"gdn_kernel_amd/{op}.py::kernel"
    assert spec["destination_passing_style"] is True
    paths = {s["path"] for s in sol["sources"]}
    assert "gdn_kernel_amd/csrc/gdn_prefill.hip" in paths and "include/gdn_kernel_amd.h" in paths
    for s in sol["sources"]:
        assert s["content"] == (ROOT / s["path"]).read_text()


def test_config_errors(tmp_path):
    bad = tmp_path / "bad.toml"
    bad.write_text('[solution]\nname = "x"\n')
    with pytest.raises(ValueError, match="definition"):
        pack.load_config(bad)
    with pytest.raises(FileNotFoundError):
        pack.load_config(tmp_path / "missing.toml")
    cfg = pack.load_config(pack.CONFIG_DIR / "decode.toml")
    cfg["build"]["files"] = cfg["build"]["files"] + ["gdn_kernel_amd/nope.hip"]
    with pytest.raises(FileNotFoundError, match="nope.hip"):
        pack.pack_solution(cfg, ROOT)
    cfg = pack.load_config(pack.CONFIG_DIR / "decode.toml")
    cfg["build"]["entry_point"] = "elsewhere.py::kernel"
    with pytest.raises(ValueError, match="entry point"):
        pack.pack_solution(cfg, ROOT)


def test_extract_refuses_escaping_paths(tmp_path):
    with pytest.raises(ValueError, match="outside"):
        pack.extract_solution({"sources": [{"path": "../evil.py", "content": ""}]}, tmp_path)


def test_extracted_tree_builds_and_exports_the_c_abi(tmp_path):
    sol = pack.pack_solution(pack.CONFIG_DIR / "prefill.toml", ROOT)
    pack.extract_solution(sol, tmp_path / "x")
    for s in sol["sources"]:
        assert (tmp_path / "x" / s["path"]).read_text() == s["content"]
    res = subprocess.run([sys.executable, "-m", "gdn_kernel_amd.build"], cwd=tmp_path / "x",
                         capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    lib = ctypes.CDLL(str(tmp_path / "x" / "gdn_kernel_amd" / "libgdn_kernel_amd.so"))
    header = (ROOT / "include" / "gdn_kernel_amd.h").read_text()
    for name in re.findall(r"^\w[\w\s\*]*?\b(gdn_\w+)\(", header, re.M):
        assert hasattr(lib, name), name
    # the extracted tree's build carries the id of its inputs, which are this tree's
    from gdn_kernel_amd import build
    lib.gdn_build_id.restype = ctypes.c_char_p
    assert lib.gdn_build_id().decode() == build.source_digest(tmp_path / "x") == build.source_digest()
