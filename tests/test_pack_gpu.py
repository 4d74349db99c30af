"""The packed solutions run on the GPU: each of solutions/{decode,prefill}.toml is packed
into a solution.json and extracted into a fresh directory, as the harness does
(scripts/pack_solution.py:36-106, then scripts/run_local.py:101-117 loads and runs
the solution).  The extracted build inputs hash to the build id of the library built
in this tree (gdn_build_id), so that library is the extracted solution's build (the
CPU test test_pack.py::test_extracted_tree_builds_and_exports_the_c_abi compiles an
extracted tree itself and finds the same id); it is placed in the extracted package,
and a fresh child process imports the solution's own entry point from there and runs
a small decode or prefill case, which is checked against the oracle here."""
import json
import shutil
import subprocess
import sys

import numpy as np
import pytest
import torch

from gdn_kernel_amd import _lib, build, pack, workloads
from tests.conftest import assert_close
from tests.gpu_util import (OUT_ATOL, OUT_RTOL, STATE_ATOL, STATE_RTOL, oracle_decode,
                            oracle_prefill, say)

pytestmark = pytest.mark.gpu

# Run in the child: import the solution's entry point from the extracted tree, call it
# destination-passing on the saved inputs, save the outputs.
CHILD = r"""
import importlib, sys
from pathlib import Path
import numpy as np, torch
root, entry, inp, outp = sys.argv[1:]
root = Path(root).resolve()
sys.path.insert(0, str(root))
mod_file, fn = entry.split("::")
mod = importlib.import_module(mod_file[:-3].replace("/", "."))
lib_mod = importlib.import_module("gdn_kernel_amd._lib")
assert root in Path(mod.__file__).resolve().parents, mod.__file__
assert root in Path(lib_mod.LIB_PATH).resolve().parents, lib_mod.LIB_PATH
kernel = getattr(mod, fn)
z = np.load(inp)
dev = torch.device("cuda:0")
t = {k: torch.from_numpy(z[k]).to(dev) for k in z.files}
for k in ("q", "k", "v", "a", "b"):
    t[k] = t[k].view(torch.bfloat16)
out = torch.full(t["v"].shape, float("nan"), dtype=torch.bfloat16, device=dev)
ns = torch.full(t["state"].shape[:1] + t["state"].shape[1:], float("nan"), device=dev)
scale = float(z["scale"])
if "cu_seqlens" in t:
    kernel(t["q"], t["k"], t["v"], t["state"], t["A_log"], t["a"], t["dt_bias"], t["b"],
           t["cu_seqlens"], scale, out, ns)
else:
    kernel(t["q"], t["k"], t["v"], t["state"], t["A_log"], t["a"], t["dt_bias"], t["b"],
           scale, out, ns)
torch.cuda.synchronize()
np.savez(outp, out=out.float().cpu().numpy(), state=ns.cpu().numpy())
print("child: ran", entry, "from", mod.__file__, flush=True)
"""


def _save_inputs(path, w):
    arrs = {}
    for k in ("q", "k", "v", "a", "b"):
        arrs[k] = w[k].contiguous().view(torch.int16).numpy()
    for k in ("state", "A_log", "dt_bias"):
        arrs[k] = w[k].numpy()
    if "cu_seqlens" in w:
        arrs["cu_seqlens"] = w["cu_seqlens"].numpy()
    arrs["scale"] = np.float64(w["scale"])
    np.savez(path, **arrs)


@pytest.mark.parametrize("op", ["decode", "prefill"])
def test_packed_solution_runs_on_the_gpu(gpu, tmp_path, op):
    lib = _lib.load()
    sol = pack.pack_solution(pack.CONFIG_DIR / f"{op}.toml")
    (tmp_path / "solution.json").write_text(json.dumps(sol))
    root = tmp_path / "solution"
    pack.extract_solution(tmp_path / "solution.json", root)
    assert build.source_digest(root) == lib.gdn_build_id().decode(), \
        "the in-tree library was not built from the packed sources (rebuild)"
    shutil.copy2(_lib.LIB_PATH, root / "gdn_kernel_amd" / _lib.LIB_PATH.name)
    if op == "decode":
        w = workloads.decode_inputs(4, seed=61, gate="slow", state_scale=0.5)
        o_ref, s_ref = oracle_decode(w)
    else:
        w = workloads.prefill_inputs([70, 9, 130], seed=62, gate="slow", state_scale=0.5)
        o_ref, s_ref = oracle_prefill(w)
    _save_inputs(tmp_path / "in.npz", w)
    say(f"packed {op} solution: running {sol['spec']['entry_point']} in a child process")
    res = subprocess.run([sys.executable, "-c", CHILD, str(root), sol["spec"]["entry_point"],
                          str(tmp_path / "in.npz"), str(tmp_path / "out.npz")],
                         cwd=tmp_path, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    say(res.stdout.strip())
    got = np.load(tmp_path / "out.npz")
    assert_close(got["out"].astype(np.float64), o_ref, OUT_RTOL, OUT_ATOL, "output")
    assert_close(got["state"].astype(np.float64), s_ref, STATE_RTOL, STATE_ATOL, "new_state")
