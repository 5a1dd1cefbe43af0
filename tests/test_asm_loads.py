"""Static check of every kernel that issues loads from inline assembly.

Kernels that issue K-loop loads from inline assembly and wait for them with
explicit `s_waitcnt vmcnt(N)` hide from the compiler that those registers
are still being written.  If register allocation ever moved or reused a
load's destination before its wait (a copy to another register, a spill, a
reuse for another value), the late load data would land in a register that
now holds something else.  This test compiles every source of the library
for gfx950, finds each kernel whose body holds a vector load between
;;#ASMSTART and ;;#ASMEND, and scans it: between such a load and the
`s_waitcnt vmcnt` that retires it, no other instruction may read or write the
load's destination registers.
"""

from __future__ import annotations

import importlib
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))

LOAD_RE = re.compile(r"^(global_load_dword(?:x[234])?|buffer_load_dword(?:x[234])?)\s+(\S+?),")
VMEM_RE = re.compile(r"^(global_|buffer_|flat_|scratch_)")
REG_RE = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+))")


def _regs(text: str) -> set[tuple[str, int]]:
    out = set()
    for m in REG_RE.finditer(text):
        kind = m.group(1)
        if m.group(4) is not None:
            out.add((kind, int(m.group(4))))
        else:
            out.update((kind, r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def check_kernel(lines: list[str]) -> list[str]:
    """Linear scan over one kernel.  Every vector-memory instruction takes a
    place in the in-order vmcnt queue; `s_waitcnt vmcnt(N)` retires all but
    the N most recent.  The destinations of loads issued from inline assembly
    (between ;;#ASMSTART and ;;#ASMEND) are protected until retired: any other
    instruction that names one of those registers is reported."""
    queue: list[tuple[int, set]] = []  # (line index, protected registers) in issue order
    problems = []
    in_asm = False
    for i, raw in enumerate(lines):
        if ";;#ASMSTART" in raw:
            in_asm = True
        if ";;#ASMEND" in raw:
            in_asm = False
        ins = raw.split(";")[0].strip()
        if not ins or ins.endswith(":") or ins.startswith("."):
            continue
        m = re.match(r"s_waitcnt\b.*vmcnt\((\d+)\)", ins)
        if m:
            n = int(m.group(1))
            queue = queue[len(queue) - n:] if n < len(queue) else queue
            continue
        if ins.startswith("s_waitcnt"):
            continue
        lm = LOAD_RE.match(ins)
        touched = _regs(ins)
        for j, d in queue:
            if d & touched:
                problems.append(f"line {i}: {ins} touches registers of the load at line {j}: {lines[j].strip()}")
        if VMEM_RE.match(ins):
            queue.append((i, _regs(lm.group(2)) if (lm and in_asm) else set()))
    return problems


def _device_asm(source: str) -> str:
    b = importlib.import_module("15642_moe_amd.build")
    res = subprocess.run([b._hipcc(), *b.compile_flags(), "-S", "--cuda-device-only", str(b.CSRC / source),
                          "-o", "-"], capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return res.stdout


def _kernels(asm: str):
    """(mangled name, body lines) of every function in one translation unit."""
    funcs = re.split(r"\n(_Z\S+):", asm)
    for k in range(1, len(funcs), 2):
        yield funcs[k], funcs[k + 1].split(".Lfunc_end")[0].split("\n")


def has_asm_load(lines: list[str]) -> bool:
    """Whether a vector-memory load sits between ;;#ASMSTART and ;;#ASMEND."""
    in_asm = False
    for raw in lines:
        if ";;#ASMSTART" in raw:
            in_asm = True
        elif ";;#ASMEND" in raw:
            in_asm = False
        elif in_asm and LOAD_RE.match(raw.split(";")[0].strip()):
            return True
    return False


def scan_all_sources() -> dict[str, int]:
    """Every kernel of every library source that issues loads from inline
    assembly is checked (found by its asm loads, not by name); returns the
    number of such kernels per source."""
    b = importlib.import_module("15642_moe_amd.build")
    found = {}
    for source in b.SOURCES:
        n = 0
        for name, lines in _kernels(_device_asm(source)):
            if not has_asm_load(lines):
                continue
            problems = check_kernel(lines)
            assert not problems, f"{source}: {name}:\n" + "\n".join(problems[:10])
            n += 1
        found[source] = n
    return found


HIPCC = shutil.which("hipcc") is not None or Path("/opt/rocm/bin/hipcc").exists()


@pytest.mark.skipif(not HIPCC, reason="hipcc not available")
def test_every_asm_load_keeps_its_registers():
    found = scan_all_sources()
    print(f"kernels with inline-asm loads per source: {found}")
    # the known users must be among them, so a change that hid their asm
    # loads from the scan (e.g. a new asm spelling) fails here
    assert found["gemm.hip"] >= 4  # decode stages 1 and 2, one or two fragments per pass
    assert found["upstream.hip"] >= 1  # router_quant_kernel


def test_checker_flags_a_moved_destination():
    """The scan must catch the failure it exists for: a load's destination
    copied (here to an accumulation register) before the wait that retires it."""
    bad = [";;#ASMSTART", "global_load_dwordx4 v[0:3], v248, s[16:17]", ";;#ASMEND",
           "v_accvgpr_write_b32 a54, v0",
           "s_waitcnt vmcnt(0)"]
    good = [";;#ASMSTART", "global_load_dwordx4 v[0:3], v248, s[16:17]",
            "global_load_dwordx4 v[4:7], v248, s[18:19]", ";;#ASMEND",
            "s_waitcnt vmcnt(1)",
            "v_accvgpr_write_b32 a54, v0"]
    assert check_kernel(bad)
    assert not check_kernel(good)
    # kernels are selected by their asm loads: a compiler-issued load alone
    # does not select one, an asm load under any kernel name does
    assert has_asm_load(bad) and has_asm_load(good)
    assert not has_asm_load(["global_load_dwordx4 v[0:3], v248, s[16:17]", "s_waitcnt vmcnt(0)"])
