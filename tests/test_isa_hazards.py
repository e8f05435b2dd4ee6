"""The compiled gfx950 code of the kernels that copy global -> LDS through inline assembly
(`global_load_lds_dwordx4` in csrc/flash_fwd.hip and csrc/gemm.hip).

On this architecture a vector-memory instruction that reads an SGPR written by a VALU
instruction (v_readfirstlane_b32, v_readlane_b32, ...) needs 5 wait states in between,
or it may read the SGPR's old value.  The compiler pads that for the memory instructions
it emits itself, but not for inline assembly, so a copy whose base address arrives that
way can read from a stale address.  These tests compile the sources as the library is
built (device code only, to assembly) and check every memory instruction's SGPR
operands: their last writer within the 5 instructions before must not be a VALU
instruction.  CPU only: hipcc cross-compiles for gfx950 here.
"""
import importlib.util
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "wan2-ti2v-5b_amd")
CSRC = os.path.join(PKG, "csrc")
WAIT_STATES = 5
MEM_PREFIXES = ("global_", "buffer_", "scratch_", "flat_")


def _build_module():
    spec = importlib.util.spec_from_file_location("wan_build", os.path.join(PKG, "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _sgprs(tok):
    m = re.match(r"s\[(\d+):(\d+)\]$", tok)
    if m:
        return {f"s{k}" for k in range(int(m.group(1)), int(m.group(2)) + 1)}
    return {tok} if re.match(r"(s\d+|m0)$", tok) else set()


def instructions(asm_text):
    """(kernel, instruction) pairs of an assembly listing, comments and directives dropped."""
    out, kernel = [], None
    for line in asm_text.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            kernel = m.group(1)
        s = line.split(";")[0].strip()
        if s and not s.startswith(".") and not s.endswith(":"):
            out.append((kernel, s))
    return out


def valu_sgpr_hazards(ins):
    """Memory instructions reading an SGPR whose last writer is a VALU instruction fewer
    than WAIT_STATES instructions before (every instruction counts as one wait state)."""
    found = []
    for i, (kernel, s) in enumerate(ins):
        parts = s.split()
        if not parts[0].startswith(MEM_PREFIXES):
            continue
        toks = [t.rstrip(",") for t in parts[1:]]
        # loads: the first operand is the destination; stores and atomics read all
        srcs = set()
        for t in (toks[1:] if "load" in parts[0] else toks):
            srcs |= _sgprs(t)
        # a global -> LDS copy also reads m0 (its LDS destination), an implicit operand
        if "_lds_" in parts[0]:
            srcs.add("m0")
        for r in srcs:
            for j in range(i - 1, max(-1, i - WAIT_STATES - 1), -1):
                p = ins[j][1].split()
                if len(p) > 1 and r in _sgprs(p[1].rstrip(",")):
                    if p[0].startswith("v_") and i - j <= WAIT_STATES:
                        found.append((kernel, ins[j][1], s, i - j))
                    break
    return found


def test_scanner_finds_a_planted_hazard():
    planted = instructions("""
_Zk:
    v_readfirstlane_b32 s12, v66
    v_readfirstlane_b32 s13, v67
    s_mov_b32 m0, s15
    s_nop 0
    global_load_lds_dwordx4 v193, s[12:13]
""")
    assert [h[3] for h in valu_sgpr_hazards(planted)]
    padded = instructions("""
_Zk:
    v_readfirstlane_b32 s12, v66
    v_readfirstlane_b32 s13, v67
    s_nop 4
    s_nop 0
    s_nop 0
    s_nop 0
    s_nop 0
    s_nop 0
    global_load_lds_dwordx4 v193, s[12:13]
""")
    assert not valu_sgpr_hazards(padded)
    # an SALU write after the VALU one is the value the load reads
    rewritten = instructions("""
_Zk:
    v_readlane_b32 s9, v255, 1
    s_add_u32 s8, s4, s8
    s_addc_u32 s9, s5, s9
    s_nop 0
    global_load_lds_dwordx4 v185, s[8:9]
""")
    assert not valu_sgpr_hazards(rewritten)
    # m0 is an implicit operand of a global -> LDS copy: a VALU write of m0 counts
    m0_valu = instructions("""
_Zk:
    v_readfirstlane_b32 m0, v12
    s_nop 0
    global_load_lds_dwordx4 v193, s[12:13]
""")
    assert [h[3] for h in valu_sgpr_hazards(m0_valu)] == [2]
    m0_salu = instructions("""
_Zk:
    v_readfirstlane_b32 s20, v12
    s_nop 4
    s_nop 4
    s_nop 4
    s_nop 4
    s_mov_b32 m0, s20
    s_nop 0
    global_load_lds_dwordx4 v193, s[12:13]
""")
    assert not valu_sgpr_hazards(m0_salu)


def _sources_with_inline_memory_asm():
    """Every source file whose inline assembly names a vector memory instruction."""
    out = []
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".hip", ".h")):
            with open(os.path.join(CSRC, name)) as f:
                text = f.read()
            if re.search(r'asm\s*(volatile\s*)?\(\s*"[^"]*(global|buffer|scratch|flat)_(load|store|atomic)', text):
                out.append(name)
    return out


SCANNED = ["flash_fwd.hip", "gemm.hip"]


def test_every_inline_memory_asm_source_is_scanned():
    # equality: a new source with such assembly must join the scan, and the search
    # must still find the two that have it
    assert _sources_with_inline_memory_asm() == SCANNED


@pytest.mark.parametrize("src", SCANNED)
def test_no_valu_sgpr_write_before_a_memory_read(src, tmp_path):
    build = _build_module()
    if not os.path.exists(build.HIPCC) and shutil.which("hipcc") is None:
        pytest.skip("hipcc is not installed")
    out = tmp_path / (src + ".s")
    cmd = [build.HIPCC, *[f for f in build.DEVICE_FLAGS if f != "-fPIC"], "-I", CSRC,
           "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o", str(out)]
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert p.returncode == 0, p.stdout[-2000:]
    ins = instructions(out.read_text())
    assert any(s.startswith("global_load_lds_dwordx4") for _, s in ins)
    hazards = valu_sgpr_hazards(ins)
    assert not hazards, hazards[:5]
