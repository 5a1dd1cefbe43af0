"""Static check of every kernel that issues loads from inline assembly.

Kernels that issue K-loop loads from inline assembly and wait for them with
explicit `s_waitcnt vmcnt(N)` hide from the compiler that those registers
are still being written.  If register allocation ever moved or reused a
load's destination before its wait (a copy to another register, a spill, a
reuse for another value), the late load data would land in a register that
now holds something else.  This test compiles every source of the library
for gfx950, finds each kernel whose body holds a vector load between
;;#ASMSTART and ;;#ASMEND, and checks it: on every path through the
kernel's control flow (branches and loop back-edges, whatever order the
compiler lays the blocks out in), between such a load and the
`s_waitcnt vmcnt` that retires it, no other instruction may read or write
the load's destination registers; and no such load may, on any path, be
issued with more vector-memory instructions in flight than the 6-bit vmcnt
counter holds (63), since the explicit waits count on it.
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


LABEL_RE = re.compile(r"^(\.LBB\w+):")
BRANCH_RE = re.compile(r"^(s_branch|s_cbranch_\w+)\s+(\.LBB\w+)")
END_RE = re.compile(r"^(s_endpgm|s_setpc_b64|s_trap)\b")
WAIT_RE = re.compile(r"s_waitcnt\b.*vmcnt\((\d+)\)")
VMCNT_MAX = 63  # gfx950's vmcnt field is 6 bits
MAX_QUEUE = 72  # older entries fold into the last position


def _instructions(lines: list[str]):
    """(line index, instruction text, inside inline asm, label) per line that
    holds an instruction or a label."""
    in_asm = False
    for i, raw in enumerate(lines):
        if ";;#ASMSTART" in raw:
            in_asm = True
        if ";;#ASMEND" in raw:
            in_asm = False
        ins = raw.split(";")[0].strip()
        m = LABEL_RE.match(ins)
        if m:
            yield i, "", in_asm, m.group(1)
            continue
        if not ins or ins.endswith(":") or ins.startswith("."):
            continue
        yield i, ins, in_asm, None


def _blocks(lines: list[str]):
    """Basic blocks of one kernel body: a list of (instructions, successor
    block indices), instructions as (line index, text, inside inline asm)."""
    blocks, labels = [], {}
    cur: list = []
    term: list = []  # per block: (branch target label or None, falls through)

    def close(target, falls):
        blocks.append(cur)
        term.append((target, falls))

    for i, ins, in_asm, label in _instructions(lines):
        if label is not None:
            if cur:
                close(None, True)
                cur = []
            labels[label] = len(blocks)
            continue
        cur.append((i, ins, in_asm))
        b = BRANCH_RE.match(ins)
        if b:
            close(b.group(2), b.group(1) != "s_branch")
            cur = []
        elif END_RE.match(ins):
            close(None, False)
            cur = []
    if cur:
        close(None, False)
    succ = []
    for k, (target, falls) in enumerate(term):
        s = []
        if target is not None and target in labels:
            s.append(labels[target])
        if falls and k + 1 < len(blocks):
            s.append(k + 1)
        succ.append(s)
    return list(zip(blocks, succ))


def _merge(a: tuple, b: tuple) -> tuple:
    n = max(len(a), len(b))
    return tuple((a[k] if k < len(a) else frozenset()) | (b[k] if k < len(b) else frozenset()) for k in range(n))


def _transfer(state: tuple, block, problems=None) -> tuple:
    """The vmcnt queue after one block.  state[k] is the set of registers
    protected by the k-th youngest outstanding vector-memory instruction
    (over every path that reaches the block, so a register is flagged if any
    path may still be loading it)."""
    for i, ins, in_asm in block:
        m = WAIT_RE.match(ins)
        if m:
            state = state[:int(m.group(1))]
            continue
        if ins.startswith("s_waitcnt"):
            continue
        if problems is not None:
            touched = _regs(ins)
            for k, d in enumerate(state):
                if d & touched:
                    problems.append(f"line {i}: {ins} touches registers of a load still in flight "
                                    f"({k} younger vector-memory instructions)")
        if VMEM_RE.match(ins):
            lm = LOAD_RE.match(ins)
            state = (frozenset(_regs(lm.group(2))) if (lm and in_asm) else frozenset(),) + state
            if problems is not None and lm and in_asm and len(state) > VMCNT_MAX:
                problems.append(f"line {i}: {ins} may be the {len(state)}th vector-memory instruction in "
                                f"flight: vmcnt counts to {VMCNT_MAX}, so the waits that follow under-count")
            if len(state) > MAX_QUEUE:
                state = state[:MAX_QUEUE - 1] + (frozenset().union(*state[MAX_QUEUE - 1:]),)
    return state


def check_kernel(lines: list[str]) -> list[str]:
    """Dataflow over the kernel's basic blocks.  Every vector-memory
    instruction takes a place in the in-order vmcnt queue; `s_waitcnt
    vmcnt(N)` retires all but the N most recent.  The destinations of loads
    issued from inline assembly (between ;;#ASMSTART and ;;#ASMEND) are
    protected until retired: any other instruction that names one of those
    registers on some path is reported.  Queue states meeting at a block are
    merged position by position (k-th youngest with k-th youngest), which
    over-approximates every path, loops included (iterated to a fixpoint)."""
    blocks = _blocks(lines)
    if not blocks:
        return []
    state_in = [None] * len(blocks)
    state_in[0] = ()
    work = [0]
    while work:
        k = work.pop()
        out = _transfer(state_in[k], blocks[k][0])
        for s in blocks[k][1]:
            new = out if state_in[s] is None else _merge(state_in[s], out)
            if new != state_in[s]:
                state_in[s] = new
                work.append(s)
    problems: list[str] = []
    for k, (block, _) in enumerate(blocks):
        if state_in[k] is not None:
            _transfer(state_in[k], block, problems)
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


def test_checker_flags_more_loads_in_flight_than_vmcnt_holds():
    """A ring that issues its next K-block's loads while NR-1 K-blocks are
    still in flight must keep all of them within vmcnt's 63: 8 K-blocks of 9
    loads (72) are flagged, 8 of 7 (56) are not."""
    def ring(lpk, nr):
        lines = []
        for k in range(lpk * nr):
            lines += [";;#ASMSTART", f"global_load_dword v{k % 200}, v248, s[16:17]", ";;#ASMEND"]
        return lines + [f"s_waitcnt vmcnt({lpk * (nr - 1)})", "s_endpgm"]
    assert any("vmcnt counts to 63" in p for p in check_kernel(ring(9, 8)))
    assert not check_kernel(ring(7, 8))


def test_checker_follows_control_flow():
    """Hazards that only a path through a branch or a loop back-edge shows
    are flagged; a safe loop whose latch block is laid out before its header
    is not."""
    load = [";;#ASMSTART", "global_load_dwordx4 v[0:3], v248, s[16:17]", ";;#ASMEND"]
    # back-edge: the load at the loop bottom, its register read at the top
    loop = [".LBB0_1:", "v_add_u32_e32 v5, v0, v5", *load, "s_cbranch_scc1 .LBB0_1", "s_endpgm"]
    assert check_kernel(loop)
    # the same loop waiting at the top is fine
    loop_ok = [".LBB0_1:", "s_waitcnt vmcnt(0)", "v_add_u32_e32 v5, v0, v5", *load,
               "s_cbranch_scc1 .LBB0_1", "s_waitcnt vmcnt(0)", "s_endpgm"]
    assert not check_kernel(loop_ok)
    # one path skips the wait
    branch = [*load, "s_cbranch_scc0 .LBB0_2", "s_waitcnt vmcnt(0)", ".LBB0_2:", "v_mov_b32_e32 v9, v1"]
    assert check_kernel(branch)
    # latch laid out before the header (entry branches over it): the wait in
    # the header runs before the use in the latch on every path
    rotated = [*load, "s_branch .LBB0_3", ".LBB0_2:", "v_mov_b32_e32 v9, v1", *load,
               ".LBB0_3:", "s_waitcnt vmcnt(0)", "s_cbranch_scc1 .LBB0_2", "s_endpgm"]
    assert not check_kernel(rotated)
