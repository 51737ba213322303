"""Instruction-level guard over the built library's gfx950 code: no vector
store of more than 8 bytes has a data register overwritten by the next
VALU instructions.

A 12/16-byte buffer store reads its data registers after it issues. The ISA
documents one wait state before a VALU may overwrite them, except for a
buffer store whose scalar offset is a register, so the compiler inserts
nothing there. On gfx950 such a store (``buffer_store_dwordx4 v[12:15], ...,
s2 offen``) followed at once by ``v_perm_b32 v12, ...`` now and then stored
the new value in lanes 12..15 of each row of 16 lanes. The kernels now give
every such store a constant scalar offset, which the compiler's wait-state
rule covers; this test disassembles the shipped code object (CPU only) and
fails on any store whose data is overwritten within two instructions.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "strict_amd" / "libstrict_hip.so"
OBJDUMP = Path("/opt/rocm/llvm/bin/llvm-objdump")

_STORE = re.compile(r"^(buffer|global|flat)_store_dwordx([34])\s+(.*)$")
_VREG = re.compile(r"v\[(\d+):(\d+)\]|v(\d+)")


def _regs(tok: str):
    m = _VREG.fullmatch(tok.strip())
    if not m:
        return None
    if m.group(3) is not None:
        r = int(m.group(3))
        return r, r
    return int(m.group(1)), int(m.group(2))


def store_data_overwrites(asm_lines, window: int = 2):
    """(store, overwriting instruction, distance) for every >8-byte vector store
    whose data registers a VALU instruction writes within ``window``
    instructions (an ``s_nop`` in between ends the window)."""
    insts = []
    for line in asm_lines:
        t = line.split("//")[0].split(";")[0].strip()
        if not t or t.endswith(":") or t.startswith("."):
            continue
        insts.append(t)
    found = []
    for i, t in enumerate(insts):
        m = _STORE.match(t)
        if not m:
            continue
        ops = [o.strip() for o in m.group(3).split(",")]
        data = _regs(ops[0] if m.group(1) == "buffer" else ops[1])
        if data is None:
            continue
        for d in range(1, window + 1):
            if i + d >= len(insts):
                break
            nxt = insts[i + d]
            if nxt.startswith("s_nop"):
                break
            if not nxt.startswith("v_"):
                continue
            parts = nxt.split(None, 1)
            if len(parts) < 2:
                continue
            dst = _regs(parts[1].split(",")[0])
            if dst and not (dst[1] < data[0] or dst[0] > data[1]):
                found.append((t, nxt, d))
    return found


def test_scanner_flags_the_pattern_and_passes_the_fix():
    bad = """
        buffer_store_dwordx4 v[12:15], v38, s[12:15], s2 offen nt
        v_perm_b32 v12, 0, v8, v39
    """.splitlines()
    near = """
        buffer_store_dwordx4 v[8:11], v40, s[12:15], s2 offen nt
        s_lshl_b32 s2, s2, 2
        v_perm_b32 v9, 0, v22, v42
    """.splitlines()
    fixed = """
        buffer_store_dwordx4 v[12:15], v30, s[8:11], 0 offen nt
        buffer_load_dwordx4 v[12:15], v37, s[4:7], s2 offen
        v_add_u32_e32 v16, v12, v13
    """.splitlines()
    padded = """
        global_store_dwordx4 v[4:5], v[6:9], off
        s_nop 0
        v_mov_b32_e32 v6, 0
    """.splitlines()
    other = """
        buffer_store_dwordx4 v[12:15], v30, s[8:11], s2 offen
        v_cmp_eq_u32_e32 vcc, v12, v13
        v_add_u32_e32 v16, v12, v13
    """.splitlines()
    assert len(store_data_overwrites(bad)) == 1
    assert store_data_overwrites(near)[0][2] == 2
    assert store_data_overwrites(fixed) == []
    assert store_data_overwrites(padded) == []
    assert store_data_overwrites(other) == []


def test_built_library_has_no_store_data_overwrite(tmp_path):
    if not LIB.exists():
        pytest.skip("libstrict_hip.so not built")
    if not OBJDUMP.exists():
        pytest.skip("llvm-objdump not installed")
    lib = tmp_path / "lib.so"
    shutil.copy(LIB, lib)
    subprocess.run([str(OBJDUMP), "--offloading", str(lib)], check=True, cwd=tmp_path,
                   capture_output=True)
    objs = sorted(tmp_path.glob("lib.so.*gfx950"))
    assert objs, "no gfx950 code object in the library"
    found, stores = [], 0
    for obj in objs:
        dis = subprocess.run([str(OBJDUMP), "-d", "--no-show-raw-insn", str(obj)], check=True,
                             capture_output=True, text=True).stdout
        stores += len(re.findall(r"_store_dwordx[34]\s", dis))
        found += store_data_overwrites(dis.splitlines())
    assert stores > 100, f"only {stores} wide stores disassembled"
    assert not found, "\n".join(f"{s}  ->  {n} (distance {d})" for s, n, d in found[:10])
