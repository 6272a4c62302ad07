"""A packed solution runs on the GPU: solution.json of each definition is
unpacked into a fresh directory, given the library built in this tree (so the
GPU box compiles nothing), and its entry point -- imported from the unpacked
tree in a child process -- is checked against the oracle on seeded inputs.
Tolerance as everywhere (conftest.py): bf16 output atol = rtol = 1e-2; f32
state atol = 1e-3 * max|state_ref|.
"""

import json
import os
import shutil
import subprocess
import sys

import numpy as np
import pytest

from conftest import PKG, assert_output_close, assert_state_close
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

from gdn_amd import _lib, packing  # noqa: E402

CHILD = r"""
import json, sys
import numpy as np
args = json.loads(sys.argv[1])
sys.path.insert(0, args["pkg"])
from gdn_amd import packing
doc = packing.read_solution(args["json"])
for m in [m for m in sys.modules if m == "gdn_amd" or m.startswith("gdn_amd.")]:
    del sys.modules[m]
sys.path.remove(args["pkg"])
fn = packing.load_entry(doc, args["dest"])
import torch
import gdn_amd._lib as L
assert L.LIB_PATH.startswith(args["dest"]), L.LIB_PATH
dev = torch.device("cuda", 0)
inp = dict(np.load(args["inputs"]))
t = {}
for n, x in inp.items():
    x = torch.from_numpy(x).to(dev)
    t[n] = x.to(torch.bfloat16) if n in ("q", "k", "v", "a", "b") else x
scale = float(inp["scale"])
if args["kind"] == "decode":
    B, hv = t["v"].shape[0], t["v"].shape[2]
    out = torch.empty((B, 1, hv, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((B, hv, 128, 128), dtype=torch.float32, device=dev)
    fn(t["q"], t["k"], t["v"], t["state"], t["A_log"], t["a"], t["dt_bias"], t["b"], scale,
       out, ns)
else:
    T, hv = t["v"].shape[0], t["v"].shape[1]
    N = t["cu_seqlens"].numel() - 1
    out = torch.empty((T, hv, 128), dtype=torch.bfloat16, device=dev)
    ns = torch.empty((N, hv, 128, 128), dtype=torch.float32, device=dev)
    fn(t["q"], t["k"], t["v"], t["state"], t["A_log"], t["a"], t["dt_bias"], t["b"],
       t["cu_seqlens"], scale, out, ns)
torch.cuda.synchronize()
np.savez(args["outputs"], o=out.float().cpu().numpy(), s=ns.cpu().numpy())
print("child done", flush=True)
"""


@pytest.mark.parametrize("definition", ["gdn_decode_qk4_v8_d128_k_last",
                                        "gdn_prefill_qk4_v8_d128_k_last"])
def test_packed_solution_runs_and_matches_oracle(cuda_device, tmp_path, definition):
    print(f"packed solution {definition}", flush=True)
    doc = packing.pack_solution(definition)
    js = packing.write_solution(doc, tmp_path / "solution.json")
    dest = tmp_path / "unpacked"
    packing.unpack_solution(doc, dest)
    shutil.copy2(_lib.LIB_PATH, dest / "gated-delta-network_amd" / "gdn_amd")
    if "decode" in definition:
        kind, inp = "decode", O.make_decode_inputs(3, seed=70)
        o_ref, s_ref = O.decode(**inp)
    else:
        kind, inp = "prefill", O.make_prefill_inputs([70, 5, 0, 130], seed=71)
        o_ref, s_ref = O.prefill_seq_c(**inp)
    np.savez(tmp_path / "in.npz", **{k: np.asarray(v) for k, v in inp.items()})
    args = dict(pkg=PKG, json=str(js), dest=str(dest.resolve()), kind=kind,
                inputs=str(tmp_path / "in.npz"), outputs=str(tmp_path / "out.npz"))
    r = subprocess.run([sys.executable, "-c", CHILD, json.dumps(args)], capture_output=True,
                       text=True, timeout=300, env=dict(os.environ, PYTHONUNBUFFERED="1"))
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-3000:]
    res = np.load(tmp_path / "out.npz")
    assert_output_close(res["o"], o_ref)
    assert_state_close(res["s"], s_ref)
