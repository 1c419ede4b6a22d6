"""The gfx950 assembly of every kernel source, scanned for wait-state hazards that the
compiler cannot see.  The LDS-DMA copies (global_load_lds_dwordx4) are issued from inline asm
(csrc/common.h: dma16, dma16_at), so the compiler's hazard recognizer does not look at them:

  * a VALU instruction that writes an SGPR (v_readfirstlane_b32, v_readlane_b32, v_cmp ...)
    followed by a VMEM instruction that reads that SGPR needs 5 wait states (gfx9 family);
  * an SALU write of M0 followed by an LDS DMA needs 1 (the asm's own s_nop 0 gives it).

The copies' scalar base operands are meant to come from scalar arithmetic on kernel
arguments; if a change ever makes the compiler produce one with v_readfirstlane right before
a copy, the copy would read a stale address.  This test compiles each csrc/*.hip to assembly
(no GPU needed) and fails on any such sequence."""

import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "flicker_amd", "csrc")
VMEM = ("global_load", "global_store", "buffer_load", "buffer_store", "global_atomic")


def _sregs(tok: str) -> set:
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"s(\d+)", tok)
    return {int(m.group(1))} if m else set()


def hazards(asm: str) -> list:
    """(kind, writer, reader) for every VMEM / LDS-DMA instruction reading an SGPR written by
    a VALU instruction fewer than 5 wait states before it, or M0 written by SALU with none."""
    ins = []
    for line in asm.splitlines():
        line = line.split(";")[0].strip()
        if line and not line.endswith(":") and not line.startswith((".", "#")):
            ins.append(line)
    found = []
    for i, line in enumerate(ins):
        op = line.split()[0]
        if not op.startswith(VMEM):
            continue
        used = set()
        for tok in line[len(op):].split(","):
            used |= _sregs(tok.strip())
        waits = 0
        # the 12 instructions before it in program order (across branches too: a conservative
        # reading, since a fall-through or loop back edge may join them)
        for j in range(i - 1, max(-1, i - 12), -1):
            prev = ins[j]
            pop = prev.split()[0]
            if pop == "s_nop":
                waits += int(prev.split()[1]) + 1
                continue
            if pop == "s_endpgm":
                break
            dst = prev[len(pop):].split(",")[0].strip() if "," in prev else ""
            if pop.startswith("v_") and waits < 5 and _sregs(dst) & used:
                found.append(("VALU SGPR write -> VMEM read", prev, line))
            if "lds" in op and dst == "m0" and pop.startswith("s_") and waits < 1:
                found.append(("SALU M0 write -> LDS DMA", prev, line))
            waits += 1
    return found


def test_scanner_finds_a_planted_hazard():
    """The scanner itself: a v_readfirstlane feeding a copy's address one wait state later is
    flagged; the same sequence with 5 wait states, or with an SALU producer, is not."""
    bad = "v_readfirstlane_b32 s8, v46\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v1, s[8:9]\n"
    ok = "v_readfirstlane_b32 s8, v46\n\ts_nop 4\n\tglobal_load_lds_dwordx4 v1, s[8:9]\n"
    salu = "s_add_u32 s8, s8, s4\n\tglobal_load_lds_dwordx4 v1, s[8:9]\n"
    m0 = "s_mov_b32 m0, s7\n\tglobal_load_lds_dwordx4 v1, s[8:9]\n"
    assert [h[0] for h in hazards(bad)] == ["VALU SGPR write -> VMEM read"]
    assert hazards(ok) == [] and hazards(salu) == []
    assert [h[0] for h in hazards(m0)] == ["SALU M0 write -> LDS DMA"]


@pytest.mark.parametrize("source", sorted(f for f in os.listdir(CSRC) if f.endswith(".hip")))
def test_kernel_assembly_has_no_hidden_hazards(source):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    from flicker_amd.build import ARCH, DEVICE_FLAGS
    with tempfile.TemporaryDirectory() as tmp:
        out = os.path.join(tmp, source + ".s")
        cmd = [hipcc, "-O3", "-std=c++17", f"--offload-arch={ARCH}", f"-I{os.path.join(ROOT, 'include')}",
               f"-I{CSRC}", *DEVICE_FLAGS, "--cuda-device-only", "-S", os.path.join(CSRC, source), "-o", out]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        assert proc.returncode == 0, proc.stderr[-2000:]
        asm = open(out).read()
    found = hazards(asm)
    assert not found, "\n".join(f"{k}: {w!r} -> {r!r}" for k, w, r in found[:10])
