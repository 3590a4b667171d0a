"""Static checks of the built library's gfx950 code, without a GPU.

Kernels whose arguments span several scalar-cache lines touch every line at
their start with one inline-assembly statement (``kernarg_lines`` in
``csrc/gr_common.h``): N scalar loads off the kernel-argument pointer, then
one wait.  A load's destination register is written when the load returns,
so none may be a register of the base pointer that the statement's later
loads still read: a fast return would hand them a data word as their
address.  The compiler chooses the registers per instantiation (the outputs
are early-clobber so it may not reuse the inputs'); this test reads the
disassembly of every kernel in the library and checks each such sequence.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "vllm-gr-ehaleva_amd", "vllm_gr_amd", "_lib", "libgr_beam.so")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"

LOAD = re.compile(r"^\s+s_load_dword\s+s(\d+),\s*s\[(\d+):(\d+)\],\s*(0x[0-9a-f]+|0)\s")


READELF = "/opt/rocm/llvm/bin/llvm-readelf"


def _code_objects(tool_args):
    """Run an LLVM tool over every gfx950 code object in the library."""
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    if not (os.path.exists(OBJDUMP) and os.path.exists(READELF)):
        pytest.skip("LLVM tools not available")
    with tempfile.TemporaryDirectory() as d:
        lib = os.path.join(d, "lib.so")
        shutil.copy(LIB, lib)
        subprocess.run([OBJDUMP, "--offloading", lib], cwd=d, check=True, capture_output=True)
        objs = sorted(os.path.join(d, f) for f in os.listdir(d) if "amdgcn" in f)
        assert objs, "no gfx950 code object in the library"
        return "\n".join(subprocess.run(tool_args + [o], check=True, capture_output=True,
                                        text=True).stdout for o in objs)


def _disassembly():
    return _code_objects([OBJDUMP, "-d"])


def _scratch_sizes():
    """Kernel name -> private segment (scratch) bytes per lane, from the code
    objects' metadata notes."""
    out, name = {}, None
    for line in _code_objects([READELF, "--notes"]).split("\n"):
        m = re.match(r"^\s+\.name:\s+(\S+)", line)
        if m:
            name = m.group(1)
        m = re.match(r"^\s+\.private_segment_fixed_size:\s+(\d+)", line)
        if m and name:
            out[name] = int(m.group(1))
    return out


def _touch_sequences(text):
    """(kernel, base pair, destinations) of every run of scalar loads at
    offsets 0, 0x40, 0x80, ... off one base pair."""
    lines = text.split("\n")
    kernel, out = None, []
    for i, line in enumerate(lines):
        m = re.match(r"^[0-9a-f]+ <(.*)>:", line)
        if m:
            kernel = m.group(1)
            continue
        m = LOAD.match(line)
        if not m or int(m.group(4), 16) != 0:
            continue
        base = (int(m.group(2)), int(m.group(3)))
        dests, k = [], i
        while k < len(lines):
            mm = LOAD.match(lines[k])
            if not mm or (int(mm.group(2)), int(mm.group(3))) != base or int(mm.group(4), 16) != 0x40 * len(dests):
                break
            dests.append(int(mm.group(1)))
            k += 1
        if len(dests) >= 2:
            out.append((kernel, base, dests))
    return out


def test_kernel_argument_touch_never_loads_into_its_base():
    seqs = _touch_sequences(_disassembly())
    kernels = {k for k, _, _ in seqs}
    # the decode / prefill kernel (every instantiation), the split merge, the
    # fork and the prune merges all carry the touch
    assert any("decode_mfma" in k for k in kernels) and any("split_merge" in k for k in kernels)
    assert any("beam_fork" in k for k in kernels) and any("prune_merge" in k for k in kernels)
    bad = [(k, b, d) for k, b, d in seqs if any(b[0] <= x <= b[1] for x in d)]
    assert not bad, bad[:4]


def test_touch_check_flags_an_overlap():
    """The check itself: a planted sequence whose first destination is the
    base's low register is reported."""
    text = ("0000000000001000 <kern>:\n"
            "\ts_load_dword s0, s[0:1], 0x0   // 000000001000: C0020000 00000000\n"
            "\ts_load_dword s3, s[0:1], 0x40  // 000000001008: C00200C0 00000040\n"
            "\ts_load_dword s4, s[0:1], 0x80  // 000000001010: C0020100 00000080\n")
    seqs = _touch_sequences(text)
    assert seqs == [("kern", (0, 1), [0, 3, 4])]
    assert any(seqs[0][1][0] <= x <= seqs[0][1][1] for x in seqs[0][2])


def test_attention_kernels_keep_no_stack():
    """The decode / prefill kernel keeps its row state in registers: no step
    lambda is left out of line (one that is takes what it captures by
    reference -- O, Q, the row state -- through a per-lane stack in scratch:
    1.7 KB per lane in the soft-capped prefill, 11x slower), the plain
    128-dim kernels (no soft cap, window, ALiBi or fp8) use no scratch at
    all and the soft-capped and head-pair (head_dim 64) ones at most a few
    spilled registers."""
    text = _disassembly()
    out_of_line = sorted(set(re.findall(r"<(_ZZN2gr\S*decode_mfma\S*)>:", text)))
    assert not out_of_line, out_of_line[:4]
    sizes = _scratch_sizes()
    # decode_mfma<DT, SOFTCAP, PREFILL, SPLIT, OPT, KV8, PAIR>: OPT = KV8 = false
    plain = {k: v for k, v in sizes.items() if re.search(r"decode_mfmaILi[12]ELb[01]ELb[01]ELb[01]ELb0ELb0E", k)}
    assert len(plain) >= 12, sorted(plain)
    assert all(v <= 64 for v in plain.values()), {k: v for k, v in plain.items() if v > 64}
    nocap = {k: v for k, v in plain.items() if re.search(r"decode_mfmaILi[12]ELb0ELb[01]ELb[01]ELb0ELb0ELb0E", k)}
    assert len(nocap) >= 6, sorted(nocap)
    assert all(v == 0 for v in nocap.values()), {k: v for k, v in nocap.items() if v}


def test_path_kernels_outside_attention_keep_no_stack():
    """The pruning, fork and split-merge kernels of the decode step hold
    their state in registers and LDS: none of them touches scratch (the
    very wide requests' one-pass merge, which keeps 16 candidates per thread,
    is the exception and is not checked)."""
    sizes = _scratch_sizes()
    names = ("prune_rows", "prune_merge_part", "prune_merge_lists", "beam_fork", "beam_append",
             "split_merge", "catalog_advance")
    found = {k: v for k, v in sizes.items() if any(n in k for n in names)}
    for n in names:
        assert any(n in k for k in found), n
    assert all(v == 0 for v in found.values()), {k: v for k, v in found.items() if v}
