"""Checks on the gfx950 assembly of the kernels (CPU only: hipcc
cross-compiles).

A vector store wider than 64 bits whose data registers are overwritten by
the very next VALU instruction was seen on MI355X to store a wrong first
dword now and then; the compiler placed no wait state there.  The store
helpers add wait states; this test keeps every kernel free of that pattern.
Also: no packed-FP32 instructions (built with -packed-fp32-ops)."""
import os
import re
import subprocess
import tempfile

import pytest

from orthossm_amd import build as B

WIDE_STORE = re.compile(r"^(buffer|global|flat)_store_dword(x3|x4)\s+(.*)$")
VREG = re.compile(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b")


def regs(op):
    out = set()
    for m in VREG.finditer(op):
        if m.group(3):
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def instructions(asm):
    for line in asm.splitlines():
        t = line.strip()
        if line.startswith("\t") and t and not t.startswith((".", ";")):
            yield t


def hazards(asm):
    """(store, next) pairs where the instruction right after a >64-bit store
    is a VALU writing one of the store's data registers."""
    ins = list(instructions(asm))
    found = []
    for k, t in enumerate(ins[:-1]):
        m = WIDE_STORE.match(t)
        if not m:
            continue
        ops = [o.strip() for o in re.split(r",(?![^\[]*\])", m.group(3))]
        # data operand: first for buffer stores, second for global/flat stores
        data = regs(ops[0] if m.group(1) == "buffer" else ops[1])
        nxt = ins[k + 1]
        if nxt.startswith("v_") and not nxt.startswith(("v_cmp", "v_readfirstlane", "v_readlane")):
            dst = nxt.split(None, 1)[1].split(",")[0] if " " in nxt else ""
            if regs(dst) & data:
                found.append((t, nxt))
    return found


@pytest.fixture(scope="module")
def kernels_asm():
    out = {}
    with tempfile.TemporaryDirectory() as d:
        for src in B.sources():
            name = os.path.basename(src)
            dst = os.path.join(d, name + ".s")
            subprocess.run(B.device_asm_command(src, dst), check=True, capture_output=True)
            out[name] = open(dst).read()
    return out


def test_hazard_detector_flags_the_pattern():
    asm = "\tbuffer_store_dwordx4 v[74:77], v114, s[4:7], s2 offen nt\n\tv_med3_f32 v74, v70, v72, v73\n"
    assert len(hazards(asm)) == 1
    ok = "\tbuffer_store_dwordx4 v[74:77], v114, s[4:7], s2 offen nt\n\ts_nop 1\n\tv_med3_f32 v74, v70, v72, v73\n"
    assert hazards(ok) == []
    glob = "\tglobal_store_dwordx4 v[70:71], v[6:9], off\n\tv_mov_b32_e32 v7, 0\n"
    assert len(hazards(glob)) == 1
    addr_only = "\tglobal_store_dwordx4 v[70:71], v[6:9], off\n\tv_mov_b32_e32 v70, 0\n"
    assert hazards(addr_only) == []


def test_no_wide_store_data_overwritten_by_next_valu(kernels_asm):
    for name, asm in kernels_asm.items():
        assert hazards(asm) == [], (name, hazards(asm)[:3])


def test_no_packed_fp32(kernels_asm):
    for name, asm in kernels_asm.items():
        assert not re.search(r"\bv_pk_(add|mul|fma|mov)_f32\b", asm), name
