"""Host-side logic of the Python entry points (no GPU needed): argument
resolution and validation happen before anything reaches the C ABI."""

import math

import pytest
import torch

from gdn_amd import _common, decode, prefill


def test_resolve_scale_follows_reference():
    assert _common.resolve_scale(None) == 1 / math.sqrt(128)
    assert _common.resolve_scale(0.0) == 1 / math.sqrt(128)
    assert _common.resolve_scale(torch.tensor(0.5)) == 0.5
    assert _common.resolve_scale(2) == 2.0
    for bad in (-1.0, float("inf"), float("nan")):
        with pytest.raises(ValueError):
            _common.resolve_scale(bad)


def _decode_cpu_args(B=2):
    bf, f = torch.bfloat16, torch.float32
    return [torch.zeros(B, 1, 4, 128, dtype=bf), torch.zeros(B, 1, 4, 128, dtype=bf),
            torch.zeros(B, 1, 8, 128, dtype=bf), torch.zeros(B, 8, 128, 128, dtype=f),
            torch.zeros(8, dtype=f), torch.zeros(B, 1, 8, dtype=bf), torch.zeros(8, dtype=f),
            torch.zeros(B, 1, 8, dtype=bf), 1.0, torch.zeros(B, 1, 8, 128, dtype=bf),
            torch.zeros(B, 8, 128, 128, dtype=f)]


def test_decode_rejects_host_tensors():
    with pytest.raises(ValueError, match="device"):
        decode.kernel(*_decode_cpu_args())


def test_decode_rejects_bad_shapes_before_device_check():
    args = _decode_cpu_args()
    args[0] = torch.zeros(2, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="q must be"):
        decode.kernel(*args)


def test_prefill_rejects_host_tensors_and_bad_cu():
    bf, f = torch.bfloat16, torch.float32
    T = 10
    args = [torch.zeros(T, 4, 128, dtype=bf), torch.zeros(T, 4, 128, dtype=bf),
            torch.zeros(T, 8, 128, dtype=bf), None, torch.zeros(8, dtype=f),
            torch.zeros(T, 8, dtype=bf), torch.zeros(8, dtype=f), torch.zeros(T, 8, dtype=bf),
            torch.tensor([0, T]), 1.0, torch.zeros(T, 8, 128, dtype=bf),
            torch.zeros(1, 8, 128, 128, dtype=f)]
    with pytest.raises(ValueError, match="device"):
        prefill.kernel(*args)


def test_fast_ok_rejects_non_tensors_and_mismatches():
    t = torch.zeros(2, 3)
    assert not _common.fast_ok((t,), (torch.float32,), ((2, 3),))  # host tensor
    assert not _common.fast_ok((None,), (torch.float32,), ((2, 3),))


def test_bench_script_imports_and_refuses_more_gpus():
    # bench.py's helpers and profiling workloads exist; --gpus N > 1 exits 2
    # before touching a device
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, root)
    import bench
    for name in ("bench_decode", "bench_prefill", "bench_prefill_rotated", "bench_prefill_clone",
                 "bench_copy", "_dev_inputs", "measured_traffic", "measured_mfma", "main"):
        assert callable(getattr(bench, name)), name
    assert "decode_b64" in bench.ONLY_WORKLOADS and "prefill_1x8192" in bench.ONLY_WORKLOADS
    t = bench.Timing([3.0, 1.0, 2.0, 5.0, 4.0])
    assert (t.ms, t.lo, t.hi, t.n) == (3.0, 1.0, 5.0, 5)
    # the committed counter summaries name the kernel sources they were
    # measured on, and are read only while the tree's sources match
    for f in ("decode_b64_hbm_traffic.md", "prefill_mfma_counters.md", "prefill_hbm_traffic.md"):
        with open(os.path.join(root, "profiles", f)) as fh:
            assert any(ln.startswith("kernel_sources_sha16: ") for ln in fh), f
    sha = bench.kernel_sources_sha16()
    assert len(sha) == 16 and int(sha, 16) >= 0
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        cur, old = os.path.join(d, "cur.md"), os.path.join(d, "old.md")
        body = "traffic_bytes_per_launch: 123\nmfma_util.x.call: 0.5\n"
        with open(cur, "w") as fh:
            fh.write(f"kernel_sources_sha16: {sha}\n" + body)
        with open(old, "w") as fh:
            fh.write("kernel_sources_sha16: 0123456789abcdef\n" + body)
        assert bench.measured_traffic(cur) == 123
        assert bench.measured_mfma(cur) == {"mfma_util.x.call": 0.5}
        assert bench.measured_traffic(old) is None and bench.measured_mfma(old) is None
        assert bench.measured_traffic(os.path.join(d, "absent.md")) is None
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
