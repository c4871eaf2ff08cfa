"""Checks gfx950 assembly for registers touched while a load into them is in
flight.

A ``global_load_dwordx4 vDST, ...`` written as inline asm completes
asynchronously; the kernel tracks it with ``s_waitcnt vmcnt(n)``, which waits
until at most n memory operations are outstanding.  Memory operations retire
in issue order on this target, so a load is complete after ``vmcnt(n)`` when
at least n memory operations were issued after it.  Reading, copying or
overwriting its destination registers before such a wait is a hazard.

The scan follows the text in order and, when it meets a backward branch the
first time, walks the loop body once more with the state it has (so loads
issued near a loop's end and used at its top are checked too).  Forward
branches fall through.  It is a conservative reading of straight-line code,
sized to the grouped GEMM kernels, not a general control-flow analysis.
"""
import re

VMEM = re.compile(r"^\s*(global_|buffer_|scratch_|flat_)")
LOAD_DST = re.compile(r"^\s*global_load_dwordx?\d*\s+(v\[\d+:\d+\]|v\d+)\s*,")
WAIT = re.compile(r"^\s*s_waitcnt\b.*?\bvmcnt\((\d+)\)")
LABEL = re.compile(r"^(\.LBB\w+):")
BRANCH = re.compile(r"^\s*s_(?:c)?branch\w*\s+(\.LBB\w+)")


def _regs(text):
    out = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b", text):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def _body(line):
    return line.split(";")[0].rstrip()


def check(asm_text, max_steps=2_000_000):
    """List of (line number, instruction, load line number) hazards."""
    lines = asm_text.split("\n")
    labels = {}
    for i, l in enumerate(lines):
        m = LABEL.match(l)
        if m:
            labels[m.group(1)] = i
    hazards = []
    pending = []          # [load line, dest regs, memory ops issued since]
    taken = set()         # backward branches already walked once
    i, steps = 0, 0
    while i < len(lines) and steps < max_steps:
        steps += 1
        raw = lines[i]
        line = _body(raw)
        if re.match(r"^\S.*:\s*(;.*)?$", raw) and not LABEL.match(raw):
            pending = []  # a new function
        w = WAIT.match(line)
        if w:
            n = int(w.group(1))
            pending = [p for p in pending if p[2] < n]
        elif VMEM.match(line):
            m = LOAD_DST.match(line)
            srcs = line.split(",", 1)[1] if m else line
            touched = _regs(srcs)
            for p in pending:
                if p[1] & touched:
                    hazards.append((i + 1, line.strip(), p[0]))
            for p in pending:
                p[2] += 1
            if m:
                d = _regs(m.group(1))
                pending = [p for p in pending if not (p[1] & d)] + [[i + 1, d, 0]]
        elif line.strip() and not line.strip().startswith((".", ";")):
            touched = _regs(line)
            for p in pending:
                if p[1] & touched:
                    hazards.append((i + 1, line.strip(), p[0]))
                    p[1] = p[1] - touched  # report a register once
        b = BRANCH.match(line)
        if b and b.group(1) in labels and labels[b.group(1)] < i and i not in taken:
            taken.add(i)
            i = labels[b.group(1)]
            continue
        i += 1
    return hazards
