"""Static check of gfx950 kernel assembly for in-flight inline-asm loads.

The decode page loads are inline-asm global loads whose results are waited for
later with explicit ``s_waitcnt vmcnt(N)`` (paged_decode_wg.h: gload /
wait_page). The compiler does not know those registers are still being
written: if it ever copied, reused or read one before the wait that covers the
load (under register pressure, say), the kernel would silently use stale data.
This module finds any such access in compiled assembly.

Model: vector memory instructions enter one in-order queue per wave (on gfx9
``vmcnt`` counts loads and stores together and they retire in order);
``s_waitcnt vmcnt(N)`` retires the oldest entries until at most N remain. An
instruction that names a destination register of an inline-asm load still in
the queue is a hit. Every control-flow path is explored: a worklist over
(basic block, queue state) pairs, with queue states kept from the oldest pending
inline-asm load on (which changes no answer, see _canonical) so that loops reach a
fixed point; the check raises rather than give up if a block's states exceed a cap,
so a kernel that passes had every path explored.
"""

from __future__ import annotations

import re

_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
_LABEL = re.compile(r"^(\.LBB\d+_\d+):")
_BRANCH_TARGET = re.compile(r"s_(c?branch\w*)\s+(\.LBB\d+_\d+)")
_VMCNT = re.compile(r"s_waitcnt\s+(?:.*\s)?vmcnt\((\d+)\)")
_VMEM = re.compile(r"(global|buffer|scratch|flat)_(load|store|atomic)")


def registers(operands: str) -> set[tuple[str, int]]:
    """The VGPRs and AGPRs an operand string names, as (kind, index) pairs."""
    out = set()
    for m in _REG.finditer(operands):
        if m.group(1):
            out.update((m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
        else:
            out.add((m.group(4), int(m.group(5))))
    return out


def kernel_names(asm: str) -> list[str]:
    """Mangled names of the kernels defined in an assembly file."""
    return re.findall(r"^(_Z\w+):", asm, flags=re.M)


def _blocks(asm: str, name: str):
    start = re.search(r"^" + re.escape(name) + r":", asm, flags=re.M).end()
    body = asm[start:asm.index(".Lfunc_end", start)].splitlines()
    blocks, order = {"entry": []}, ["entry"]
    cur, in_asm = "entry", False
    for line in body:
        s = line.strip()
        if s == ";;#ASMSTART":
            in_asm = True
            continue
        if s == ";;#ASMEND":
            in_asm = False
            continue
        m = _LABEL.match(s)
        if m:
            cur = m.group(1)
            blocks[cur] = []
            order.append(cur)
            continue
        if not s or s[0] in ";." or s.endswith(":"):
            continue
        blocks[cur].append((s, in_asm))
        if re.match(r"s_c?branch", s):  # a conditional branch ends its block; the fall-through starts a new one
            cur = cur + "'"
            blocks[cur] = []
            order.append(cur)
    succ = {}
    for i, b in enumerate(order):
        ins = blocks[b]
        last = ins[-1][0] if ins else ""
        out = [m.group(2) for s, _ in ins for m in [_BRANCH_TARGET.match(s)] if m]
        if i + 1 < len(order) and not (last.startswith("s_branch") or last.startswith("s_endpgm")):
            out.append(order[i + 1])
        succ[b] = out
    return blocks, succ


def _canonical(q: list) -> tuple:
    """The queue from its oldest pending inline-asm load on. Dropping older entries
    changes no answer: a vmcnt(N) retires such a load when len(q) - N exceeds its
    position, and removing k entries ahead of it lowers both sides by k. With no
    inline-asm load pending, nothing in the queue matters."""
    for i, e in enumerate(q):
        if e[0]:
            return tuple(q[i:])
    return ()


def check_kernel(asm: str, name: str, max_states_per_block: int = 4096) -> list[tuple[str, str]]:
    """(block, instruction) pairs that touch a register of an inline-asm load still in flight.

    Raises RuntimeError if a block's distinct queue states exceed max_states_per_block
    (the exploration would be incomplete)."""
    blocks, succ = _blocks(asm, name)
    hits: set[tuple[str, str]] = set()
    seen: set = set()
    per_block: dict[str, int] = {}
    work = [("entry", ())]
    while work:
        b, queue = work.pop()
        if (b, queue) in seen:
            continue
        per_block[b] = per_block.get(b, 0) + 1
        if per_block[b] > max_states_per_block:
            raise RuntimeError(f"{name}: more than {max_states_per_block} queue states at {b}")
        seen.add((b, queue))
        q = list(queue)  # entries: (is an inline-asm load, its destination registers)
        for s, in_asm in blocks[b]:
            m = _VMCNT.match(s)
            if m:
                del q[:max(0, len(q) - int(m.group(1)))]
                q = list(_canonical(q))
                continue
            if s.startswith("s_waitcnt"):
                continue
            op, _, rest = s.partition(" ")
            pending = set().union(*(e[1] for e in q if e[0])) if q else set()
            if registers(rest) & pending:
                hits.add((b, s))
            if _VMEM.match(op):
                writes_regs = "load" in op and "_lds_" not in op
                dst = frozenset(registers(rest.split(",")[0])) if writes_regs else frozenset()
                q.append((in_asm and writes_regs, dst))
                q = list(_canonical(q))
        for nb in succ[b]:
            work.append((nb, tuple(q)))
    return sorted(hits)
