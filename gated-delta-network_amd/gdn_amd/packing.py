"""Solution packing: a FlashInfer-Bench ``solution.json`` for the HIP operators.

Reference: scripts/pack_solution.py:28-89 reads
solutions/<definition>/config.toml and packs the source files of
solutions/<definition>/solution/<language>/ into a Solution document with
flashinfer_bench (``BuildSpec`` + ``pack_solution_from_files``,
pack_solution.py:64-82).  flashinfer_bench is a third-party package that the
reference neither vendors nor pins (README.md:165 installs it unversioned) and
it is not installed here, so this module writes the document itself, with the
fields the reference fills in:

  name, definition, author       config.toml [solution] (pack_solution.py:74-76)
  spec.language, spec.entry_point,
  spec.destination_passing_style config.toml [build] (pack_solution.py:50-51, 63-69)
  spec.target_hardware           config.toml [build] target_hardware (the reference
                                 passes ["cuda"], pack_solution.py:66)
  spec.dependencies              [] (BuildSpec's package list, FAQ.md:65)
  sources                        [{path, content}], one per text file
  description                    config.toml [solution] description

The key names and nesting are those of flashinfer-bench's published Solution /
BuildSpec / SourceFile schema.  The entry point keeps the reference's
``<file>::<function>`` form (config.toml ``entry_point = "kernel.py::kernel"``).

What is packed: the solution's own directory (its ``kernel.py`` at the root of
the document) plus every file the entry point needs from this repository, at
its repository-relative path: the ``gdn_amd`` Python package, the HIP sources
and Makefile of ``csrc/``, and ``include/gdn_amd.h``.  No binary travels:
an unpacked tree builds ``libgdn_amd.so`` from those sources with hipcc on
first import (``ensure_library``), as the reference's CUDA solution compiles
itself with ``load_inline`` (solution/cuda/binding.py:181-192).
"""

from __future__ import annotations

import argparse
import fcntl
import glob
import importlib.util
import json
import os
import subprocess
import sys
from pathlib import Path, PurePosixPath

try:
    import tomllib
except ImportError:  # Python < 3.11
    import tomli as tomllib

from . import _lib

PKG_DIR = Path(__file__).resolve().parent          # .../gated-delta-network_amd/gdn_amd
REPO_ROOT = PKG_DIR.parent.parent                   # the repository root
SOLUTIONS_DIR = PKG_DIR.parent / "solutions"

# Files (globs relative to the repository root) that every HIP solution needs
# beside its own directory.
PACKAGE_FILES = (
    "gated-delta-network_amd/gdn_amd/*.py",
    "gated-delta-network_amd/csrc/*.hip",
    "gated-delta-network_amd/csrc/*.cpp",
    "gated-delta-network_amd/csrc/*.h",
    "gated-delta-network_amd/csrc/Makefile",
    "include/gdn_amd.h",
)

LANGUAGES = ("python", "triton", "cuda")
SOLUTION_KEYS = ("name", "definition", "author", "spec", "sources", "description")
SPEC_KEYS = ("language", "target_hardware", "entry_point", "dependencies",
             "destination_passing_style")


def load_config(solution_dir) -> dict:
    """config.toml of one solution folder (reference pack_solution.py:28-34)."""
    path = Path(solution_dir) / "config.toml"
    if not path.exists():
        raise FileNotFoundError(f"config file not found: {path}")
    with open(path, "rb") as f:
        return tomllib.load(f)


def _split_entry(entry_point: str):
    if not isinstance(entry_point, str) or entry_point.count("::") != 1:
        raise ValueError(f"entry_point must be '<file>::<function>', got {entry_point!r}")
    file, func = entry_point.split("::")
    if not file.endswith(".py") or not func.isidentifier():
        raise ValueError(f"entry_point must be '<file.py>::<function>', got {entry_point!r}")
    return file, func


def _read_text(path: Path) -> str:
    try:
        return path.read_text(encoding="utf-8")
    except UnicodeDecodeError as e:
        raise ValueError(f"{path}: not UTF-8 text, cannot be packed") from e


def pack_solution(definition: str, solutions_dir=SOLUTIONS_DIR, repo_root=REPO_ROOT) -> dict:
    """The Solution document of ``solutions_dir/<definition>`` as a dict."""
    solution_dir = Path(solutions_dir) / definition
    if not solution_dir.is_dir():
        have = sorted(d.name for d in Path(solutions_dir).iterdir() if d.is_dir())
        raise FileNotFoundError(f"solution directory not found: {solution_dir}; have {have}")
    config = load_config(solution_dir)
    sol, build = config["solution"], config["build"]
    language = build["language"]
    if language not in LANGUAGES:
        raise ValueError(f"unsupported language {language!r}")
    entry_file, _ = _split_entry(build["entry_point"])
    candidates = sorted(p.parent for p in (solution_dir / "solution").glob(f"*/{entry_file}"))
    if len(candidates) != 1:
        raise FileNotFoundError(
            f"expected one solution/<backend>/{entry_file} under {solution_dir}, found "
            f"{[str(c) for c in candidates]}")
    source_dir = candidates[0]

    sources = {}
    for p in sorted(source_dir.rglob("*")):
        if p.is_file() and "__pycache__" not in p.parts and p.suffix != ".pyc":
            sources[p.relative_to(source_dir).as_posix()] = _read_text(p)
    root = Path(repo_root)
    for pattern in PACKAGE_FILES:
        matched = sorted(glob.glob(str(root / pattern)))
        if not matched:
            raise FileNotFoundError(f"no file matches {pattern} under {root}")
        for m in matched:
            rel = Path(m).relative_to(root).as_posix()
            if rel in sources:
                raise ValueError(f"{rel} would be packed twice")
            sources[rel] = _read_text(Path(m))

    doc = {
        "name": sol["name"],
        "definition": sol["definition"],
        "author": sol["author"],
        "spec": {
            "language": language,
            "target_hardware": list(build.get("target_hardware", ["gfx950"])),
            "entry_point": build["entry_point"],
            "dependencies": list(build.get("dependencies", [])),
            "destination_passing_style": bool(build.get("destination_passing_style", True)),
        },
        "sources": [{"path": p, "content": c} for p, c in sources.items()],
        "description": sol.get("description"),
    }
    validate_solution(doc)
    return doc


def write_solution(doc: dict, output) -> Path:
    """Write ``doc`` as indented JSON (the reference writes
    ``model_dump_json(indent=2)``, pack_solution.py:82)."""
    out = Path(output)
    out.write_text(json.dumps(doc, indent=2, ensure_ascii=False) + "\n", encoding="utf-8")
    return out


def read_solution(path) -> dict:
    doc = json.loads(Path(path).read_text(encoding="utf-8"))
    validate_solution(doc)
    return doc


def _check_path(p: str) -> PurePosixPath:
    pp = PurePosixPath(p)
    if not p or pp.is_absolute() or ".." in pp.parts or "\\" in p or pp.as_posix() != p:
        raise ValueError(f"source path {p!r} must be a plain relative path")
    return pp


def validate_solution(doc: dict) -> None:
    """Structural checks of a Solution document; raises ValueError."""
    if not isinstance(doc, dict) or set(doc) != set(SOLUTION_KEYS):
        raise ValueError(f"a solution has exactly the keys {SOLUTION_KEYS}")
    for k in ("name", "definition", "author"):
        if not isinstance(doc[k], str) or not doc[k]:
            raise ValueError(f"solution {k} must be a non-empty string")
    if doc["description"] is not None and not isinstance(doc["description"], str):
        raise ValueError("solution description must be a string or null")
    spec = doc["spec"]
    if not isinstance(spec, dict) or set(spec) != set(SPEC_KEYS):
        raise ValueError(f"spec has exactly the keys {SPEC_KEYS}")
    if spec["language"] not in LANGUAGES:
        raise ValueError(f"unsupported language {spec['language']!r}")
    if not isinstance(spec["destination_passing_style"], bool):
        raise ValueError("destination_passing_style must be a bool")
    for k in ("target_hardware", "dependencies"):
        if not isinstance(spec[k], list) or not all(isinstance(x, str) and x for x in spec[k]):
            raise ValueError(f"spec.{k} must be a list of non-empty strings")
    if not spec["target_hardware"]:
        raise ValueError("spec.target_hardware must name at least one target")
    entry_file, _ = _split_entry(spec["entry_point"])
    seen = set()
    if not isinstance(doc["sources"], list) or not doc["sources"]:
        raise ValueError("sources must be a non-empty list")
    for s in doc["sources"]:
        if not isinstance(s, dict) or set(s) != {"path", "content"}:
            raise ValueError("each source is {path, content}")
        _check_path(s["path"])
        if not isinstance(s["content"], str):
            raise ValueError(f"{s['path']}: content must be text")
        if s["path"] in seen:
            raise ValueError(f"{s['path']} appears twice")
        seen.add(s["path"])
    if entry_file not in seen:
        raise ValueError(f"entry file {entry_file} is not among the sources")


def unpack_solution(doc: dict, dest) -> Path:
    """Write every source of ``doc`` under ``dest`` (created if needed)."""
    validate_solution(doc)
    root = Path(dest)
    root.mkdir(parents=True, exist_ok=True)
    for s in doc["sources"]:
        target = root.joinpath(*_check_path(s["path"]).parts)
        target.parent.mkdir(parents=True, exist_ok=True)
        target.write_text(s["content"], encoding="utf-8")
    return root


def load_entry(doc: dict, dest):
    """Unpack ``doc`` under ``dest`` and return its entry-point function.

    The unpacked tree brings its own ``gdn_amd`` package; load it in a process
    that has not imported another copy (checked)."""
    root = unpack_solution(doc, dest).resolve()
    entry_file, func = _split_entry(doc["spec"]["entry_point"])
    name = "gdn_solution_" + "".join(c if c.isalnum() else "_" for c in doc["name"])
    spec = importlib.util.spec_from_file_location(name, root / entry_file)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    pkg = sys.modules.get("gdn_amd")
    if pkg is None or not Path(pkg.__file__).resolve().is_relative_to(root):
        where = None if pkg is None else pkg.__file__
        raise RuntimeError(f"gdn_amd was imported from {where}, not from the unpacked "
                           f"solution under {root}; load it in a fresh process")
    return getattr(mod, func)


def ensure_library(jobs: int = 8) -> str:
    """Build libgdn_amd.so from the sources beside this package if it is not
    there yet (one builder at a time, under a file lock); return its path."""
    lib = _lib.LIB_PATH
    if os.path.exists(lib):
        return lib
    csrc = PKG_DIR.parent / "csrc"
    with open(csrc / ".build.lock", "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        if not os.path.exists(lib):
            r = subprocess.run(["make", "-C", str(csrc), f"-j{int(jobs)}"],
                               capture_output=True, text=True)
            if r.returncode != 0 or not os.path.exists(lib):
                raise RuntimeError(f"building {lib} failed:\n{r.stdout[-4000:]}\n"
                                   f"{r.stderr[-4000:]}")
    return lib


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Pack a solution folder into solution.json")
    ap.add_argument("definition", help="folder under solutions/, e.g. "
                    "gdn_decode_qk4_v8_d128_k_last, or 'all'")
    ap.add_argument("-o", "--output", type=Path, default=None,
                    help="output path (default: solutions/<definition>/solution.json)")
    args = ap.parse_args(argv)
    names = (sorted(d.name for d in SOLUTIONS_DIR.iterdir() if (d / "config.toml").exists())
             if args.definition == "all" else [args.definition])
    if args.output is not None and len(names) != 1:
        ap.error("-o needs a single definition")
    for n in names:
        doc = pack_solution(n)
        out = write_solution(doc, args.output or SOLUTIONS_DIR / n / "solution.json")
        print(f"packed {out}: {doc['name']} ({doc['definition']}), "
              f"{len(doc['sources'])} sources, language {doc['spec']['language']}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
