"""Checks the gfx950 assembly of the sampling kernels for a hazard of their
explicitly issued loads.

The fast kernel issues its row and history loads through inline assembly
and waits for them with explicit `s_waitcnt vmcnt(N)` (lmrs_amd/csrc/
fast_bf16.hpp).  The compiler does not know such a load is outstanding: if
it reads, copies or reuses a destination register before the wait that
covers the load, the data is wrong or a later value is overwritten when the
load lands.

The scanner follows each kernel's control flow: basic blocks split at labels
and branches, successors from `s_branch`, the `s_cbranch_*` family (taken
and fall-through), long branches (`s_getpc_b64` / `s_add_u32` with the
target label / `s_setpc_b64`) and `s_endpgm`.  The state at a block is the
set of queues of outstanding vector-memory operations that some path into it
can leave (each `s_waitcnt vmcnt(N)` keeps the N youngest), and every
instruction that names a destination register of an outstanding
inline-assembly load on some path is reported.  A queue only needs the
operations from its oldest inline-assembly load on (older ones do not change
when it retires), and never more than 63 of them (the counter's limit), which
keeps the states of loops finite.
"""
from __future__ import annotations

import re

_REG = re.compile(r"\bv(\d+)\b|\bv\[(\d+):(\d+)\]")
_LABEL = re.compile(r"^(\.?[A-Za-z_][\w.$]*):")
_VM_OPS = ("global_", "buffer_", "scratch_", "flat_")
_MAX_QUEUE = 63


def _regs(text: str) -> frozenset[int]:
    out: set[int] = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out.add(int(m.group(1)))
        else:
            out.update(range(int(m.group(2)), int(m.group(3)) + 1))
    return frozenset(out)


def kernel_names(asm: str, prefix: str) -> list[str]:
    return [m.group(1) for m in re.finditer(r"^(" + re.escape(prefix) + r"\w*):", asm, re.M)]


def _normalise(q: tuple) -> tuple:
    """Drops the operations older than the oldest inline-assembly load and
    those beyond the hardware's 63 outstanding."""
    q = q[-_MAX_QUEUE:]
    for i, (_, dst) in enumerate(q):
        if dst:
            return q[i:]
    return ()


def _parse(asm: str, kernel: str):
    """The kernel's instructions (line, text, op, in_asm) and label -> index."""
    lines = asm.split("\n")
    start = next(i for i, ln in enumerate(lines) if ln.startswith(kernel + ":"))
    ins, labels, in_asm = [], {}, False
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
        m = _LABEL.match(raw)
        if m:
            labels[m.group(1)] = len(ins)
            continue
        text = raw.split(";")[0].strip()
        if not text or text.startswith("."):
            continue
        ins.append((i, text, text.split()[0], in_asm))
    return lines, ins, labels


def _successors(ins, labels, k: int) -> list[int]:
    _, text, op, _ = ins[k]
    nxt = [k + 1] if k + 1 < len(ins) else []
    target = lambda t: labels[t]  # noqa: E731  (a missing label is a parse error: KeyError)
    if op == "s_endpgm":
        return []
    if op == "s_branch":
        return [target(text.split()[1])]
    if op.startswith("s_cbranch_"):
        return nxt + [target(text.split()[1])]
    if op == "s_setpc_b64":
        # a long branch: the target label is in the s_add_u32 a few instructions before
        for j in range(k - 1, max(-1, k - 6), -1):
            m = re.search(r"\((\.?[\w.$]+)-\.Lpost_getpc\w*\)", ins[j][1])
            if m:
                return [target(m.group(1))]
        raise ValueError(f"s_setpc_b64 without a recognised target at line {ins[k][0] + 1}")
    return nxt


def scan(asm: str, kernel: str) -> list[str]:
    """Hazards of `kernel` (its mangled name) in the assembly text."""
    lines, ins, labels = _parse(asm, kernel)
    if not ins:
        return []
    # basic blocks: leaders are the entry, label targets and instructions after a branch
    leaders = {0} | set(labels.values())
    for k, (_, _, op, _) in enumerate(ins):
        if op.startswith(("s_branch", "s_cbranch_", "s_setpc", "s_endpgm")) and k + 1 < len(ins):
            leaders.add(k + 1)
    leaders = sorted(x for x in leaders if x < len(ins))
    block_end = {b: e for b, e in zip(leaders, leaders[1:] + [len(ins)])}
    states: dict[int, set] = {0: {()}}
    done: dict[int, set] = {}
    work = [0]
    found: dict[int, str] = {}
    while work:
        b = work.pop()
        todo = states[b] - done.get(b, set())
        if not todo:
            continue
        done.setdefault(b, set()).update(todo)
        out = set()
        for q in todo:
            for k in range(b, block_end[b]):
                line, text, op, in_asm = ins[k]
                if op == "s_waitcnt":
                    m = re.search(r"vmcnt\((\d+)\)", text)
                    if m:
                        n = int(m.group(1))
                        q = q[len(q) - n:] if n < len(q) else q
                        q = _normalise(q)
                    continue
                used = _regs(text[len(op):])
                for ln, dst in q:
                    if dst and used & dst and line not in found:
                        found[line] = f"line {line + 1}: {text}  (outstanding: {lines[ln].strip()})"
                        break
                if op.startswith(_VM_OPS):
                    dst = _regs(text[len(op):].split(",")[0]) if ("load" in op and in_asm) else None
                    q = _normalise(q + ((line, dst),))
            out.add(q)
        last = block_end[b] - 1
        for s in _successors(ins, labels, last):
            new = out - done.get(s, set())
            if new - states.get(s, set()):
                states.setdefault(s, set()).update(new)
                work.append(s)
    return [found[k] for k in sorted(found)]
