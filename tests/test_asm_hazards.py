"""Hazard check of the hand-issued buffer loads in the generated gfx950 code.

The GEMM's and the router's LDS DMA (``buffer_load_dwordx4 ... lds``) and the
router's x loads are issued from inline assembly, so the compiler's hazard
recognizer does not protect them. gfx9 needs 5 wait
states between a VALU write of an SGPR (``v_readfirstlane``, ``v_readlane``,
``v_cmp`` into an SGPR pair) and a VMEM instruction reading that SGPR. The
buffer descriptor comes from such writes, and ``v_readlane`` also restores
spilled SGPRs. A load that reads a stale descriptor base can fault. This test
compiles the kernel sources to assembly and checks every buffer load in every
instantiation (the compiler's own loads pass by construction).
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SRCS = [ROOT / "parallel_amd" / "csrc" / name for name in ("grouped_gemm.hip", "router.hip")]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

_SGPR = re.compile(r"s\[(\d+):(\d+)\]|s(\d+)\b")


def _sgprs(text):
    regs = set()
    for m in _SGPR.finditer(text):
        if m.group(1) is not None:
            regs.update(range(int(m.group(1)), int(m.group(2)) + 1))
        else:
            regs.add(int(m.group(3)))
    return regs


def dma_hazards(asm_lines, window=5):
    """(line, writer, load) triples where a VALU SGPR write precedes a buffer
    load reading that SGPR (its descriptor) by fewer than `window` wait states
    in straight-line code."""
    found = []
    for n, line in enumerate(asm_lines):
        text = line.strip()
        if not text.startswith("buffer_load"):
            continue
        operands = text.split(None, 1)[1].split(",")
        rsrc = next((_sgprs(o) for o in operands[1:] if o.strip().startswith("s")), set())
        waits, k = 0, n - 1
        while k >= 0 and waits < window:
            prev = asm_lines[k].strip()
            k -= 1
            if not prev or prev.startswith((";", ".")):
                continue
            if prev.endswith(":"):
                continue  # a label: keep walking back through the fall-through path (conservative)
            mnemonic = prev.split()[0]
            if mnemonic == "s_nop":
                waits += int(prev.split()[1], 0) + 1
                continue
            if mnemonic.startswith(("v_readfirstlane", "v_readlane")) or (
                mnemonic.startswith("v_cmp") and mnemonic.endswith("_e64")
            ):
                dst = prev.split(None, 1)[1].split(",")[0]
                if _sgprs(dst) & rsrc:
                    found.append((n, prev, text))
            waits += 1
    return found


def test_scanner_flags_a_planted_hazard():
    planted = [
        "v_readfirstlane_b32 s31, v4",
        "s_mov_b32 m0, s12",
        "buffer_load_dwordx4 v9, s[28:31], 0 offen lds",
    ]
    assert len(dma_hazards(planted)) == 1
    covered = ["v_readfirstlane_b32 s31, v4", "s_nop 4", "buffer_load_dwordx4 v9, s[28:31], 0 offen lds"]
    assert dma_hazards(covered) == []
    # a load into registers: the descriptor is the first scalar operand
    into_regs = ["v_readfirstlane_b32 s13, v4", "buffer_load_dwordx4 v[2:5], v2, s[12:15], 0 offen"]
    assert len(dma_hazards(into_regs)) == 1
    assert dma_hazards(["v_readfirstlane_b32 s13, v4", "s_nop 4", into_regs[1]]) == []


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
@pytest.mark.parametrize("src", SRCS, ids=lambda p: p.name)
def test_lds_dma_has_its_wait_states(tmp_path, src):
    asm = tmp_path / (src.stem + ".s")
    cmd = [
        HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-mcode-object-version=5",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "--cuda-device-only", "-S", str(src), "-o", str(asm),
    ]
    proc = subprocess.run(cmd, capture_output=True, text=True, cwd=ROOT)
    assert proc.returncode == 0, proc.stderr[-2000:]
    lines = asm.read_text().split("\n")
    n_dma = sum(1 for l in lines if l.strip().startswith("buffer_load") and l.strip().endswith(" lds"))
    assert n_dma > 0, "no LDS DMA found in the generated code"
    hazards = dma_hazards(lines)
    assert not hazards, "VALU SGPR write too close to an LDS DMA:\n" + "\n".join(
        f"  line {n}: {w}  ->  {l}" for n, w, l in hazards[:10]
    )
