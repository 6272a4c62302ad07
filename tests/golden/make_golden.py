"""Writes the golden fixtures of this directory (run from the repo root:
``python tests/golden/make_golden.py``).

The reference ships no golden vectors for this path, so these fixtures are the
CPU oracle's outputs (oracle/gdn_oracle.py, itself pinned by
tests/test_oracle.py) on seeded inputs.  Inputs are defined by the numpy PCG64
recipe in oracle.make_*_inputs and recorded by seed plus the SHA-256 of every
input array, so a generator change is detected instead of silently shifting
the vectors.  Expected outputs are stored in full for the output `o` and for
selected state heads, plus float64 row sums of every state row.
"""

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import gdn_oracle as O  # noqa: E402

INPUT_NAMES = ("q", "k", "v", "state", "A_log", "a", "dt_bias", "b", "cu_seqlens")


def input_digest(inp):
    h = hashlib.sha256()
    for name in INPUT_NAMES:
        x = inp.get(name)
        if x is None:
            h.update(name.encode() + b":none")
        else:
            x = np.ascontiguousarray(x)
            h.update(name.encode() + str(x.dtype).encode() + str(x.shape).encode() + x.tobytes())
    return h.hexdigest()


def decode_fixture():
    inp = O.make_decode_inputs(1, seed=0)
    o, s = O.decode_loop(**inp)
    heads = np.array([0, 5])
    return dict(kind="decode", B=1, seed=0, sha256=input_digest(inp), o=o.astype(np.float32),
                state_heads=heads, state_sel=s[0, heads], state_rowsum=s.astype(np.float64).sum(-1))


def prefill_fixture():
    lens = [5, 0, 70]
    inp = O.make_prefill_inputs(lens, seed=0, with_state=False)
    o, s = O.prefill_seq(**inp)
    heads = np.array([0, 7])
    return dict(kind="prefill", lens=np.array(lens), seed=0, sha256=input_digest(inp),
                o_bits=O.bf16_bits(o), state_seq=2, state_heads=heads, state_sel=s[2, heads],
                state_rowsum=s.astype(np.float64).sum(-1))


def main():
    for name, fx in (("decode_b1_seed0.npz", decode_fixture()),
                     ("prefill_5_0_70_seed0.npz", prefill_fixture())):
        path = os.path.join(HERE, name)
        np.savez_compressed(path, **fx)
        print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
