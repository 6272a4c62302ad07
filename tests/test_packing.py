"""The solution.json packer (gdn_amd/packing.py) on the CPU: the document's
fields against the solution folders' config.toml (the reference fills the same
fields, scripts/pack_solution.py:46-77), sources identical to the repository
files, the validator's refusals, and an unpacked tree that builds its own
libgdn_amd.so with hipcc and imports the entry point from itself.

flashinfer_bench, which owns the Solution schema, is not installed, so the
schema itself is not checked against it (the key names follow its published
Solution / BuildSpec / SourceFile models).
"""

import copy
import ctypes
import json
import os
import re
import shutil
import subprocess
import sys

import pytest

from conftest import PKG, ROOT
from gdn_amd import packing

DEFINITIONS = ["gdn_decode_qk4_v8_d128_k_last", "gdn_prefill_qk4_v8_d128_k_last"]


@pytest.mark.parametrize("definition", DEFINITIONS)
def test_pack_fields_follow_config(definition):
    doc = packing.pack_solution(definition)
    cfg = packing.load_config(os.path.join(PKG, "solutions", definition))
    assert list(doc) == list(packing.SOLUTION_KEYS)
    assert doc["definition"] == definition == cfg["solution"]["definition"]
    assert doc["name"] == cfg["solution"]["name"]
    assert doc["author"] == cfg["solution"]["author"]
    assert doc["description"] == cfg["solution"]["description"]
    spec = doc["spec"]
    assert list(spec) == list(packing.SPEC_KEYS)
    assert spec["language"] == "python"
    assert spec["entry_point"] == "kernel.py::kernel"
    assert spec["destination_passing_style"] is True
    assert spec["target_hardware"] == ["gfx950"]
    assert spec["dependencies"] == []


@pytest.mark.parametrize("definition", DEFINITIONS)
def test_pack_sources_are_the_repository_files(definition):
    doc = packing.pack_solution(definition)
    paths = [s["path"] for s in doc["sources"]]
    assert paths[0] == "kernel.py"
    want = {"include/gdn_amd.h", "gated-delta-network_amd/csrc/Makefile",
            "gated-delta-network_amd/gdn_amd/decode.py",
            "gated-delta-network_amd/gdn_amd/prefill.py",
            "gated-delta-network_amd/gdn_amd/_lib.py",
            "gated-delta-network_amd/gdn_amd/packing.py",
            "gated-delta-network_amd/csrc/gdn_decode.hip",
            "gated-delta-network_amd/csrc/gdn_prefill.hip"}
    assert want <= set(paths)
    assert not [p for p in paths if p.endswith((".so", ".o", ".pyc")) or "__pycache__" in p]
    entry_src = os.path.join(PKG, "solutions", definition, "solution", "hip", "kernel.py")
    for s in doc["sources"]:
        src = entry_src if s["path"] == "kernel.py" else os.path.join(ROOT, s["path"])
        with open(src, encoding="utf-8") as f:
            assert f.read() == s["content"], s["path"]


def test_pack_is_deterministic_and_json_round_trips(tmp_path):
    a = packing.pack_solution(DEFINITIONS[1])
    b = packing.pack_solution(DEFINITIONS[1])
    assert a == b
    out = packing.write_solution(a, tmp_path / "solution.json")
    assert packing.read_solution(out) == a
    assert json.loads(out.read_text())["spec"]["entry_point"] == "kernel.py::kernel"


def test_cli_packs_every_solution(tmp_path):
    out = tmp_path / "d.json"
    r = subprocess.run([sys.executable, os.path.join(PKG, "solutions", "pack_solution.py"),
                        DEFINITIONS[0], "-o", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert packing.read_solution(out)["definition"] == DEFINITIONS[0]


def _broken(mutate):
    doc = packing.pack_solution(DEFINITIONS[0])
    doc = copy.deepcopy(doc)
    mutate(doc)
    return doc


@pytest.mark.parametrize("name, mutate", [
    ("escaping path", lambda d: d["sources"].append({"path": "../x.py", "content": ""})),
    ("absolute path", lambda d: d["sources"].append({"path": "/tmp/x.py", "content": ""})),
    ("duplicate path", lambda d: d["sources"].append(dict(d["sources"][0]))),
    ("no entry file", lambda d: d.__setitem__("sources", d["sources"][1:])),
    ("bad entry point", lambda d: d["spec"].__setitem__("entry_point", "kernel.py:kernel")),
    ("bad language", lambda d: d["spec"].__setitem__("language", "fortran")),
    ("dps not bool", lambda d: d["spec"].__setitem__("destination_passing_style", "yes")),
    ("extra key", lambda d: d.__setitem__("extra", 1)),
    ("missing key", lambda d: d.pop("author")),
    ("binary content", lambda d: d["sources"].append({"path": "x.bin", "content": b"\0"})),
    ("no target", lambda d: d["spec"].__setitem__("target_hardware", [])),
])
def test_validate_rejects(name, mutate, tmp_path):
    doc = _broken(mutate)
    with pytest.raises(ValueError):
        packing.validate_solution(doc)
    with pytest.raises(ValueError):
        packing.unpack_solution(doc, tmp_path / "out")
    assert not (tmp_path / "x.py").exists()


def test_unknown_definition():
    with pytest.raises(FileNotFoundError):
        packing.pack_solution("gdn_decode_qk16_v32_d128_k_last")


def _header_functions():
    with open(os.path.join(ROOT, "include", "gdn_amd.h")) as f:
        text = re.sub(r"/\*.*?\*/", "", f.read(), flags=re.S)
    return sorted(set(re.findall(r"\b(gdn_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.skipif(shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="needs make and hipcc")
def test_unpacked_tree_builds_and_loads_itself(tmp_path):
    """Unpack, build with hipcc (gfx950 cross-compile) on first import, and
    check in a fresh process that the entry point comes from the unpacked
    tree and its library exports every declared symbol."""
    doc = packing.pack_solution(DEFINITIONS[1])
    dest = tmp_path / "sol"
    code = (
        "import inspect, json, sys\n"
        f"sys.path.insert(0, {PKG!r})\n"
        "from gdn_amd import packing\n"
        f"doc = packing.read_solution({str(tmp_path / 'solution.json')!r})\n"
        "for m in [m for m in sys.modules if m == 'gdn_amd' or m.startswith('gdn_amd.')]:\n"
        "    del sys.modules[m]\n"
        f"sys.path.remove({PKG!r})\n"
        f"fn = packing.load_entry(doc, {str(dest)!r})\n"
        "import gdn_amd._lib as L\n"
        "print(json.dumps({'file': inspect.getsourcefile(fn), 'lib': L.LIB_PATH,\n"
        "                  'params': list(inspect.signature(fn).parameters)}))\n"
    )
    packing.write_solution(doc, tmp_path / "solution.json")
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    info = json.loads(r.stdout.strip().splitlines()[-1])
    assert info["file"].startswith(str(dest.resolve()))
    assert info["lib"].startswith(str(dest.resolve()))
    assert info["params"][:12] == ["q", "k", "v", "state", "A_log", "a", "dt_bias", "b",
                                   "cu_seqlens", "scale", "output", "new_state"]
    lib = ctypes.CDLL(info["lib"])
    for name in _header_functions():
        assert hasattr(lib, name), name
