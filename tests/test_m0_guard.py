"""Guard for the direct global->LDS loads of the projection kernels.

dma16s/dma4s in dq8_kernels.hip write M0 (the LDS destination of
global_load_lds_*) from inline assembly.  The compiler does not know that M0
changes there, so the kernels are correct only while no compiler-generated
instruction writes M0 (a value the compiler kept in M0 would be clobbered).
This test builds the kernels' gfx950 assembly with the library's own flags
and checks that every M0 write is the first instruction of one of those
inline-assembly blocks, followed by the wait state and the LDS load."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "decider-engine_amd", "csrc")

# a scalar or lane-read instruction whose destination is m0
_M0_WRITE = re.compile(r"^\s*(s_\w+|v_readfirstlane_b32|v_readlane_b32)\s+m0\b")


def m0_violations(asm: str):
    """(line number, text) of every M0 write that is not an inline-assembly
    DMA prologue (s_mov_b32 m0; s_nop 0; global_load_lds_*), and the number
    of prologues seen."""
    bad, dma = [], 0
    lines = asm.splitlines()
    inside = False
    block = []
    for no, line in enumerate(lines, 1):
        text = line.split(";")[0].strip()
        if line.strip().startswith(";;#ASMSTART"):
            inside, block = True, []
            continue
        if line.strip().startswith(";;#ASMEND"):
            inside = False
            writes = [i for i, (_, t) in enumerate(block) if _M0_WRITE.match(t)]
            if writes:
                ok = (writes == [0] and len(block) == 3 and block[0][1].startswith("s_mov_b32 m0,")
                      and block[1][1] == "s_nop 0" and block[2][1].startswith("global_load_lds_dword"))
                if ok:
                    dma += 1
                else:
                    bad.extend(block[i] for i in writes)
            continue
        if not text:
            continue
        if inside:
            block.append((no, text))
        elif _M0_WRITE.match(text):
            bad.append((no, text))
    return bad, dma


def test_checker_flags_planted_m0_writes():
    good = (";;#ASMSTART\n\ts_mov_b32 m0, s38\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v82, s[52:53]\n;;#ASMEND\n")
    assert m0_violations(good) == ([], 1)
    # a compiler-generated write outside any inline assembly
    bad, dma = m0_violations(good + "\ts_mov_b32 m0, -1\n\tds_gws_init v0 offset:0\n")
    assert dma == 1 and [t for _, t in bad] == ["s_mov_b32 m0, -1"]
    bad, _ = m0_violations("\tv_readfirstlane_b32 m0, v3\n")
    assert len(bad) == 1
    # an inline block that writes m0 without the DMA that consumes it
    bad, dma = m0_violations(";;#ASMSTART\n\ts_mov_b32 m0, s1\n\ts_nop 0\n;;#ASMEND\n")
    assert dma == 0 and len(bad) == 1


@pytest.mark.skipif(shutil.which("make") is None or not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="needs make and hipcc to build the gfx950 assembly")
def test_no_compiler_generated_m0_write_in_the_kernels(tmp_path):
    out = tmp_path / "dq8_kernels.s"
    subprocess.run(["make", "-s", "-C", CSRC, "asm", f"ASM={out}"], check=True, capture_output=True, timeout=600)
    bad, dma = m0_violations(out.read_text())
    assert not bad, f"M0 written outside the DMA prologues: {bad[:5]}"
    # every wide, skinny and LoRA-middle DMA loop is in the assembly
    assert dma >= 100, dma
