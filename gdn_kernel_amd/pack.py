"""Pack this library into a FlashInfer-Bench ``solution.json`` and back.

The reference packs its kernel sources with scripts/pack_solution.py:36-106:
it reads ``config.toml`` ([solution] name / definition / author, [build]
language / entry_point / files / binding / destination_passing_style), builds a
``BuildSpec`` and writes a Solution JSON whose ``sources`` hold the files'
text (config.toml:1-25; README.md:137-148, 236-257).  The flashinfer_bench
package that does this is not installed here, so this module writes the same
JSON shape itself:

    {"name", "definition", "author", "description",
     "spec": {"language", "target_hardware", "entry_point", "dependencies",
              "destination_passing_style", "binding"},
     "sources": [{"path", "content"}, ...]}

and ``extract_solution`` restores the files (the counterpart of the harness's
``extract_solution_to_files``).  The configurations shipped in
``gdn_kernel_amd/solutions/`` pack the HIP sources, the C header and the Python
binding needed to build and call the decode or prefill ``kernel``; paths are
relative to the repository root, and an extracted tree builds with
``python -m gdn_kernel_amd.build``.

Usage: python -m gdn_kernel_amd.pack [--config TOML | --op decode|prefill] [-o solution.json]
       python -m gdn_kernel_amd.pack --extract solution.json --into DIR
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

try:
    import tomllib
except ImportError:  # Python < 3.11
    import tomli as tomllib

__all__ = ["load_config", "pack_solution", "extract_solution", "REPO_ROOT", "CONFIG_DIR"]

REPO_ROOT = Path(__file__).resolve().parent.parent
CONFIG_DIR = Path(__file__).resolve().parent / "solutions"


def load_config(path) -> dict:
    path = Path(path)
    if not path.exists():
        raise FileNotFoundError(f"Config file not found: {path}")
    with open(path, "rb") as f:
        cfg = tomllib.load(f)
    for section, keys in (("solution", ("name", "definition", "author")),
                          ("build", ("language", "entry_point", "files"))):
        if section not in cfg:
            raise ValueError(f"{path}: missing [{section}]")
        for k in keys:
            if k not in cfg[section]:
                raise ValueError(f"{path}: [{section}] has no {k!r}")
    return cfg


def pack_solution(config, root=REPO_ROOT, output=None) -> dict:
    """Build the Solution dict from a config (path or dict); write it to ``output``
    if given.  Every listed file must exist under ``root``."""
    cfg = load_config(config) if not isinstance(config, dict) else config
    sol, build = cfg["solution"], cfg["build"]
    root = Path(root)
    sources = []
    for rel in build["files"]:
        p = root / rel
        if not p.is_file():
            raise FileNotFoundError(f"Source file not found: {p}")
        sources.append({"path": str(Path(rel).as_posix()), "content": p.read_text()})
    entry_file = build["entry_point"].split("::")[0]
    if entry_file not in {s["path"] for s in sources}:
        raise ValueError(f"entry point file {entry_file} is not among the packed files")
    spec = {"language": build["language"],
            "target_hardware": list(build.get("target_hardware", ["rocm:gfx950"])),
            "entry_point": build["entry_point"],
            "dependencies": list(build.get("dependencies", [])),
            "destination_passing_style": bool(build.get("destination_passing_style", True))}
    if build.get("binding"):
        spec["binding"] = build["binding"]
    solution = {"name": sol["name"], "definition": sol["definition"], "author": sol["author"],
                "description": sol.get("description", "MI355X (gfx950) HIP kernels of the "
                                       "Gated DeltaNet decode / varlen chunked prefill"),
                "spec": spec, "sources": sources}
    if output is not None:
        Path(output).write_text(json.dumps(solution, indent=2))
    return solution


def extract_solution(solution, into) -> list:
    """Write a Solution's sources under ``into``; returns the written paths.  Paths
    must stay inside ``into`` (no absolute paths, no '..')."""
    if not isinstance(solution, dict):
        solution = json.loads(Path(solution).read_text())
    into = Path(into).resolve()
    written = []
    for src in solution["sources"]:
        rel = Path(src["path"])
        if rel.is_absolute() or ".." in rel.parts:
            raise ValueError(f"refusing to write outside the target: {rel}")
        dst = (into / rel).resolve()
        dst.parent.mkdir(parents=True, exist_ok=True)
        dst.write_text(src["content"])
        written.append(dst)
    return written


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="pack / extract a FlashInfer-Bench solution.json")
    g = ap.add_mutually_exclusive_group()
    g.add_argument("--config", type=Path)
    g.add_argument("--op", choices=["decode", "prefill"], default="prefill")
    ap.add_argument("-o", "--output", type=Path, default=Path("solution.json"))
    ap.add_argument("--extract", type=Path, help="solution.json to unpack")
    ap.add_argument("--into", type=Path, help="directory to unpack into")
    args = ap.parse_args(argv)
    try:
        if args.extract:
            if not args.into:
                raise ValueError("--extract needs --into")
            for p in extract_solution(args.extract, args.into):
                print(p)
            return 0
        cfg = args.config or CONFIG_DIR / f"{args.op}.toml"
        sol = pack_solution(cfg, REPO_ROOT, args.output)
    except (OSError, ValueError) as exc:
        print(f"Error: {exc}", file=sys.stderr)
        return 1
    print(f"Solution packed: {args.output}")
    print(f"  Name: {sol['name']}")
    print(f"  Definition: {sol['definition']}")
    print(f"  Author: {sol['author']}")
    print(f"  Language: {sol['spec']['language']}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
