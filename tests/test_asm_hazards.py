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

The compiler also does not know that a load issued from inline assembly is
still in flight when the statement ends: it may copy or move the destination
registers (into AGPRs, under register pressure) before the hand-written wait,
and the copy then holds whatever the register held before. The second check
follows the memory counter through each kernel and flags any instruction that
touches the destination of an inline-assembly load before a wait retires it.
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


_VGPR = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")


def _vgprs(text):
    regs = set()
    for m in _VGPR.finditer(text):
        if m.group(1) is not None:
            regs.update((m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1))
        else:
            regs.add((m.group(4), int(m.group(5))))
    return regs


def early_uses(asm_lines):
    """(line, instruction) pairs that read or write a destination register of
    a load issued from inline assembly before an ``s_waitcnt vmcnt`` retires
    that load. Memory operations retire in issue order on the vector memory
    counter, so ``vmcnt(n)`` retires all but the n youngest. The scan is
    straight-line: an unconditional branch or the end of a kernel forgets the
    loads in flight (the instruction after it is reached from elsewhere)."""
    found, pending, in_asm = [], [], False
    for n, line in enumerate(asm_lines):
        raw = line.strip()
        if raw.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if raw.startswith(";;#ASMEND"):
            in_asm = False
            continue
        text = raw.split(";")[0].strip()
        if not text or text.startswith(".") or text.endswith(":"):
            continue
        mnemonic = text.split()[0]
        operands = text[len(mnemonic):]
        if mnemonic == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", text)
            if m:
                del pending[: max(0, len(pending) - int(m.group(1)))]
            continue
        if mnemonic in ("s_branch", "s_endpgm", "s_setpc_b64"):
            pending = []
            continue
        vmem = mnemonic.startswith(("buffer_", "global_", "scratch_", "flat_"))
        parts = [o.strip() for o in operands.split(",")]
        if vmem and "load" in mnemonic and not text.endswith(" lds"):
            dst, src = _vgprs(parts[0]), _vgprs(",".join(parts[1:]))
        elif vmem:
            dst, src = set(), _vgprs(operands)
        else:
            dst, src = _vgprs(parts[0]), _vgprs(",".join(parts[1:]))
        busy = set().union(*pending) if pending else set()
        if (src | dst) & busy:
            found.append((n, text))
        if vmem:
            pending.append(dst if in_asm else set())
    return found


def test_scanner_flags_a_register_touched_before_its_wait():
    load = [";;#ASMSTART", "buffer_load_dwordx4 v[4:7], v2, s[12:15], 0 offen", ";;#ASMEND"]
    assert len(early_uses(load + ["v_accvgpr_write_b32 a9, v5"])) == 1
    assert len(early_uses(load + ["v_mov_b32_e32 v6, 0"])) == 1  # a write the load would overwrite
    assert early_uses(load + ["s_waitcnt vmcnt(0)", "v_accvgpr_write_b32 a9, v5"]) == []
    # a younger load left in flight by vmcnt(1) does not hold the older one
    two = load + [";;#ASMSTART", "buffer_load_dwordx4 v[8:11], v3, s[12:15], 0 offen", ";;#ASMEND"]
    assert early_uses(two + ["s_waitcnt vmcnt(1)", "v_mov_b32_e32 v1, v4"]) == []
    assert len(early_uses(two + ["s_waitcnt vmcnt(1)", "v_mov_b32_e32 v1, v8"])) == 1
    # the compiler's own loads are its business (it waits for them itself)
    assert early_uses(["global_load_dword v4, v[0:1], off", "v_mov_b32_e32 v1, v4"]) == []


_ASM = {}


def _assembly(src):
    """The gfx950 assembly of one source, compiled once per test session."""
    if src not in _ASM:
        import tempfile

        with tempfile.TemporaryDirectory() as tmp:
            asm = Path(tmp) / (src.stem + ".s")
            cmd = [
                HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-mcode-object-version=5",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "--cuda-device-only", "-S", str(src), "-o", str(asm),
            ]
            proc = subprocess.run(cmd, capture_output=True, text=True, cwd=ROOT)
            assert proc.returncode == 0, proc.stderr[-2000:]
            _ASM[src] = asm.read_text().split("\n")
    return _ASM[src]


def _kernels(lines):
    """(name, first line, end line) of every kernel in an assembly listing."""
    out = []
    for n, line in enumerate(lines):
        m = re.match(r"^(_Z\w+):", line)
        if m:
            end = n
            while end < len(lines) and not lines[end].strip().startswith("s_endpgm"):
                end += 1
            out.append((m.group(1), n, end + 1))
    return out


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
@pytest.mark.parametrize("src", SRCS, ids=lambda p: p.name)
def test_asm_loads_are_not_touched_before_their_wait(src):
    lines = _assembly(src)
    bad = []
    for name, start, end in _kernels(lines):
        bad += [(name, n - start, text) for n, text in early_uses(lines[start:end])]
    assert not bad, "registers of an inline-assembly load used before its wait:\n" + "\n".join(
        f"  {name[:60]} +{n}: {text}" for name, n, text in bad[:10]
    )


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not available")
@pytest.mark.parametrize("src", SRCS, ids=lambda p: p.name)
def test_lds_dma_has_its_wait_states(src):
    lines = _assembly(src)
    n_dma = sum(1 for l in lines if l.strip().startswith("buffer_load") and l.strip().endswith(" lds"))
    assert n_dma > 0, "no LDS DMA found in the generated code"
    hazards = dma_hazards(lines)
    assert not hazards, "VALU SGPR write too close to an LDS DMA:\n" + "\n".join(
        f"  line {n}: {w}  ->  {l}" for n, w, l in hazards[:10]
    )
