"""Checks the gfx950 assembly of the sampling kernels for a hazard of their
explicitly issued loads.

The fast kernel issues its row and history loads through inline assembly
and waits for them with explicit `s_waitcnt vmcnt(N)` (lmrs_amd/csrc/
fast_bf16.hpp).  The compiler does not know such a load is outstanding: if
it reads, copies or reuses a destination register before the wait that
covers the load, the data is wrong or a later value is overwritten when the
load lands.  This scanner follows each kernel in program order, keeps the
queue of outstanding vector-memory operations (retired in order by each
`s_waitcnt vmcnt`), and reports any instruction that names a destination
register of an outstanding inline-assembly load.  It ignores control flow,
which is sound for the straight-line load pass where these loads live.
"""
from __future__ import annotations

import re

_REG = re.compile(r"\bv(\d+)\b|\bv\[(\d+):(\d+)\]")


def _regs(text: str) -> set[int]:
    out: set[int] = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out.add(int(m.group(1)))
        else:
            out.update(range(int(m.group(2)), int(m.group(3)) + 1))
    return out


def kernel_names(asm: str, prefix: str) -> list[str]:
    return [m.group(1) for m in re.finditer(r"^(" + re.escape(prefix) + r"\w*):", asm, re.M)]


def scan(asm: str, kernel: str) -> list[str]:
    """Hazards of `kernel` (its mangled name) in the assembly text."""
    lines = asm.split("\n")
    start = next(i for i, ln in enumerate(lines) if ln.startswith(kernel + ":"))
    queue: list[tuple[int, set[int] | None]] = []
    found = []
    in_asm = False
    for i in range(start + 1, len(lines)):
        raw = lines[i]
        if raw.startswith(".Lfunc_end"):
            break
        if ";;#ASMSTART" in raw:
            in_asm = True
            continue
        if ";;#ASMEND" in raw:
            in_asm = False
            continue
        ins = raw.split(";")[0].strip()
        if not ins or ins.startswith(".") or ins.endswith(":"):
            continue
        op = ins.split()[0]
        if op == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", ins)
            if m:
                del queue[: max(0, len(queue) - int(m.group(1)))]
            continue
        used = _regs(ins[len(op):])
        for ln, dst in queue:
            if dst and used & dst:
                found.append(f"line {i + 1}: {ins}  (outstanding: {lines[ln].strip()})")
                break
        if op.startswith(("global_", "buffer_", "scratch_", "flat_")):
            dst = _regs(ins[len(op):].split(",")[0]) if ("load" in op and in_asm) else None
            queue.append((i, dst))
    return found
