"""Static check of this repository's own gfx950 device code: no MFMA
accumulation chain mixes instruction shapes.

On MI355X a 16x16x32 MFMA whose result fed a 16x16x16 MFMA's accumulator
directly (results in VGPRs, the dependent instruction 0-3 slots later) gave
wrong results, so every kernel keeps one shape per accumulator chain.  This
test makes that a checked property of the built code rather than a
convention: it unbundles the gfx950 code objects of the library's own build
(gated-delta-network_amd/csrc/_build/*.o) with the ROCm LLVM tools,
disassembles them, and walks each function's instructions in order (twice,
so that a hand-off across a loop's back edge is seen too), remembering for
every VGPR/AGPR which instruction last wrote it.  For every MFMA whose
accumulator operand is a register range, the last writer of each of those
registers must not be an MFMA of another shape.

CPU only: it reads compiled code built here and runs nothing on a GPU.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "gated-delta-network_amd", "csrc", "_build")
LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
OBJECTS = ["gdn_prefill.o", "gdn_block.o", "gdn_recurrent.o", "gdn_decode.o"]

_REG = re.compile(r"^([va])(\d+)$|^([va])\[(\d+):(\d+)\]$")


def _regs(operand):
    """The VGPRs/AGPRs an operand names, as ("v", n) / ("a", n) pairs."""
    m = _REG.match(operand.strip())
    if not m:
        return []
    if m.group(1):
        return [(m.group(1), int(m.group(2)))]
    kind, lo, hi = m.group(3), int(m.group(4)), int(m.group(5))
    return [(kind, r) for r in range(lo, hi + 1)]


def _writes_first_operand(mnemonic):
    """Whether an instruction's first operand is a vector register it writes
    (VALU results, loads, LDS reads, accumulator moves) rather than data or
    an address it reads (stores, LDS writes) or a scalar result."""
    if mnemonic.startswith(("s_", "v_cmp", "v_cmpx", "v_readlane", "v_readfirstlane")):
        return False
    if "store" in mnemonic or mnemonic.startswith(("ds_write", "ds_store")):
        return False
    return mnemonic.startswith(("v_", "ds_", "buffer_", "global_", "flat_", "scratch_"))


def _functions(asm):
    """(name, [(mnemonic, [operands])]) per function of llvm-objdump output."""
    funcs, name, body = [], None, []
    for line in asm.splitlines():
        head = re.match(r"^[0-9a-f]+ <(.+)>:$", line)
        if head:
            if name is not None:
                funcs.append((name, body))
            name, body = head.group(1), []
            continue
        if name is None or not line.startswith("\t"):
            continue
        text = line.split("//")[0].strip()
        if not text:
            continue
        parts = text.split(None, 1)
        ops = [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []
        body.append((parts[0], ops))
    if name is not None:
        funcs.append((name, body))
    return funcs


def _violations(funcs):
    found = {}  # (function, instruction, register) -> hand-off, once over both sweeps
    for name, body in funcs:
        last = {}
        for sweep in range(2):
            for i, (mn, ops) in enumerate(body):
                if mn.startswith("v_mfma"):
                    if len(ops) >= 4:
                        for reg in _regs(ops[3]):
                            w = last.get(reg)
                            if w is not None and w[0].startswith("v_mfma") and w[0] != mn:
                                found[(name, i, reg)] = (name, i, w[0], mn, reg)
                    for reg in _regs(ops[0]) if ops else []:
                        last[reg] = (mn, i)
                elif ops and _writes_first_operand(mn):
                    for reg in _regs(ops[0]):
                        last[reg] = (mn, i)
    return sorted(found.values())


def _disassemble(obj, tmp):
    fatbin = os.path.join(tmp, os.path.basename(obj) + ".fatbin")
    code = os.path.join(tmp, os.path.basename(obj) + ".gfx950.co")
    subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fatbin}", obj,
                    os.path.join(tmp, "scratch.o")], check=True, capture_output=True)
    subprocess.run([f"{LLVM}/clang-offload-bundler", "--type=o", "--unbundle",
                    f"--targets={TARGET}", f"--input={fatbin}", f"--output={code}"],
                   check=True, capture_output=True)
    out = subprocess.run([f"{LLVM}/llvm-objdump", "-d", "--mcpu=gfx950", code], check=True,
                         capture_output=True, text=True)
    return out.stdout


def _need_tools():
    for tool in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"):
        if not os.path.exists(os.path.join(LLVM, tool)):
            pytest.skip(f"{tool} not found under {LLVM}")


def test_checker_flags_a_mixed_chain():
    # the checker itself, on hand-written instruction lists: a 16x16x32
    # result used as a 16x16x16 accumulator is flagged, directly and across
    # a loop's back edge; a chain of one shape, a zero accumulator and an
    # intervening VALU write of the registers are not
    mixed = [("f", [("v_mfma_f32_16x16x32_bf16", ["v[0:3]", "v[4:7]", "v[8:11]", "v[0:3]"]),
                    ("v_mfma_f32_16x16x16_bf16", ["v[12:15]", "v[4:5]", "v[8:9]", "v[0:3]"])])]
    assert len(_violations(mixed)) == 4
    loop = [("f", [("v_mfma_f32_16x16x16_bf16", ["v[12:15]", "v[4:5]", "v[8:9]", "v[0:3]"]),
                   ("s_cbranch_scc1", ["label"]),
                   ("v_mfma_f32_16x16x32_bf16", ["v[0:3]", "v[4:7]", "v[8:11]", "v[0:3]"])])]
    assert _violations(loop)
    same = [("f", [("v_mfma_f32_16x16x32_bf16", ["v[0:3]", "v[4:7]", "v[8:11]", "0"]),
                   ("v_mfma_f32_16x16x32_bf16", ["v[0:3]", "v[4:7]", "v[8:11]", "v[0:3]"]),
                   ("v_mfma_f32_16x16x16_bf16", ["v[16:19]", "v[4:5]", "v[8:9]", "0"])])]
    assert not _violations(same)
    broken = [("f", [("v_mfma_f32_16x16x32_bf16", ["v[0:3]", "v[4:7]", "v[8:11]", "v[0:3]"]),
                     ("v_mul_f32_e32", ["v0", "v20", "v0"]),
                     ("v_mul_f32_e32", ["v1", "v20", "v1"]),
                     ("v_mul_f32_e32", ["v2", "v20", "v2"]),
                     ("v_mul_f32_e32", ["v3", "v20", "v3"]),
                     ("v_mfma_f32_16x16x16_bf16", ["v[12:15]", "v[4:5]", "v[8:9]", "v[0:3]"])])]
    assert not _violations(broken)
    stores = [("f", [("v_mfma_f32_16x16x32_bf16", ["v[0:3]", "v[4:7]", "v[8:11]", "v[0:3]"]),
                     ("global_store_dwordx4", ["v[0:3]", "v[20:21]", "off"]),
                     ("v_mfma_f32_16x16x16_bf16", ["v[12:15]", "v[4:5]", "v[8:9]", "v[0:3]"])])]
    assert _violations(stores), "a store reads its first operand; it must not break the chain"


@pytest.mark.parametrize("obj", OBJECTS)
def test_built_kernels_keep_one_mfma_shape_per_chain(obj, tmp_path):
    _need_tools()
    path = os.path.join(BUILD, obj)
    if not os.path.exists(path):
        pytest.skip(f"{obj} is not built (run __graft_entry__.build() first)")
    funcs = _functions(_disassemble(path, str(tmp_path)))
    n_mfma = sum(1 for _, body in funcs for mn, _ in body if mn.startswith("v_mfma"))
    if obj != "gdn_recurrent.o" and obj != "gdn_decode.o":
        assert n_mfma > 0, f"no MFMA found in {obj}: the disassembly was not parsed"
    bad = _violations(funcs)
    assert not bad, "MFMA accumulator hand-off between shapes: " + "; ".join(
        f"{f[:60]} @{i}: {a} -> {b} ({r[0]}{r[1]})" for f, i, a, b, r in bad[:10])
