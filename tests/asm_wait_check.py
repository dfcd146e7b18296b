"""Static check of the kernels' hand-counted memory waits, on gfx950 assembly.

The hot loops issue some loads as inline asm (LDS operand reads of the MFMA
stream: ``ds_read_b128``, ``ds_read_b64_tr_b16``) and wait for them later with
a counted ``s_waitcnt lgkmcnt(N)``, so that tile DMA still in flight is not
drained.  The compiler does not know that such a load writes its destination
registers asynchronously: it treats the asm output as written when the asm
block ends.  If register allocation then copies, spills or reuses one of those
registers before the counted wait has retired the load, the copy reads stale
data and the load later overwrites whatever the register holds by then.  The
results are wrong and vary from run to run.  This was seen with three
operand reads in flight instead of two: the compiler spilled a pending
destination to scratch.

``scan`` walks each function of an assembly file in order.  It keeps the
outstanding operations of each counter: LDS, scalar-memory and message ops
under lgkmcnt; vector-memory ops under vmcnt; flat ops under both.  Each
counter retires in order, and ``s_waitcnt X(N)`` leaves only the N youngest.
The walk flags any instruction that names a register an inline-asm load
still has in flight.  The walk is linear, so each branch is followed as if it
falls through.  The kernels end every stream with a full wait, so no load is
in flight across a branch.
"""

from __future__ import annotations

import re
from dataclasses import dataclass
from typing import List, Set

_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
_WAIT = re.compile(r"\b(vmcnt|lgkmcnt)\((\d+)\)")


def registers(text: str) -> Set[str]:
    """Vector and accumulation registers named in an operand list."""
    out: Set[str] = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out.update(f"{m.group(1)}{r}" for r in range(int(m.group(2)), int(m.group(3)) + 1))
        else:
            out.add(f"{m.group(4)}{m.group(5)}")
    return out


def _counters(op: str) -> List[str]:
    if op.startswith("flat_"):
        return ["vmcnt", "lgkmcnt"]
    if op.startswith(("global_", "buffer_", "scratch_")):
        return ["vmcnt"]
    if op.startswith(("ds_", "s_load", "s_buffer_load", "s_sendmsg")) or op in ("s_memtime", "s_memrealtime"):
        return ["lgkmcnt"]
    return []


def _is_load(op: str, operands: str) -> bool:
    # an LDS-DMA form (global_load_lds_*, buffer_load_* ... lds) writes LDS, not registers
    return (op.startswith(("ds_read", "ds_load", "global_load", "buffer_load", "flat_load", "scratch_load"))
            and "_lds" not in op and not re.search(r"\blds\b", operands))


@dataclass
class Hazard:
    function: str
    line: int
    text: str
    load_line: int

    def __str__(self) -> str:
        return (f"{self.function}: line {self.line} `{self.text}` names a register of the inline-asm load "
                f"at line {self.load_line} before a wait retires it")


@dataclass
class _Op:
    dest: Set[str]
    line: int
    asm: bool


def scan(asm_text: str) -> List[Hazard]:
    """Every hazard in one assembly file (see the module docstring)."""
    lines = asm_text.split("\n")
    hazards: List[Hazard] = []
    fn = None
    queues = {"vmcnt": [], "lgkmcnt": []}
    in_asm = False
    for i, raw in enumerate(lines, 1):
        t = raw.strip()
        head = re.match(r"^([A-Za-z_.$][\w.$]*):", raw)
        if head and not raw.startswith((" ", "\t")):
            label = head.group(1)
            if label.startswith(".Lfunc_end"):
                fn = None
            elif not label.startswith("."):
                fn = label
                queues = {"vmcnt": [], "lgkmcnt": []}
                in_asm = False
            continue
        if fn is None:
            continue
        if t.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if t.startswith(";;#ASMEND"):
            in_asm = False
            continue
        code = t.split(";")[0].strip()
        if not code or code.startswith("."):
            continue
        op, _, operands = code.partition(" ")
        if op == "s_waitcnt":
            for m in _WAIT.finditer(operands):
                q = queues[m.group(1)]
                keep = int(m.group(2))
                del q[:max(0, len(q) - keep)]
            continue
        if op == "s_nop":
            continue
        named = registers(operands)
        for q in queues.values():
            for pend in q:
                if pend.asm and pend.dest & named:
                    hazards.append(Hazard(fn, i, code, pend.line))
                    break
        cnt = _counters(op)
        if cnt:
            load = _is_load(op, operands)
            dest = registers(operands.split(",")[0]) if load else set()
            entry = _Op(dest, i, in_asm and load)
            for c in cnt:
                queues[c].append(entry)
    return hazards
