"""Static check of the library's gfx950 device assembly for a hazard that the
compiler does not guard inside inline assembly.

On this GPU generation a vector memory instruction (global_*, buffer_*,
scratch_*) that reads an SGPR (a saddr base, a buffer resource or offset)
needs 5 wait states after a VALU instruction wrote that SGPR (for example a
v_readfirstlane); with fewer it can read the SGPR's previous contents.  The
compiler inserts the states for the instructions it emits, but the copies and
loads of this library are inline assembly, which its hazard pass does not
inspect, so the asm blocks supply the states themselves.  ``scan_text``
checks that every path into every vector memory instruction has them: it walks
backwards through the fall-through predecessor and every branch to a label,
counting one state per instruction and N + 1 per ``s_nop N``.

Usage:  python tests/isa_check.py file.s [...]   (exit status 1 on a finding)
"""
from __future__ import annotations

import re
import sys
from dataclasses import dataclass

WAIT_STATES = 5

_SREG = re.compile(r"\bs\[(\d+):(\d+)\]|\bs(\d+)\b")
_VMEM = ("global_", "buffer_", "scratch_")
# VALU instructions whose second operand is an SGPR destination (carry-out)
_SDST2 = ("v_add_co_", "v_sub_co_", "v_subrev_co_", "v_addc_co_", "v_subb_co_", "v_subbrev_co_",
          "v_mad_u64_u32", "v_mad_i64_i32", "v_div_scale_")
_BRANCH = re.compile(r"^s_(?:c)?branch\w*\s+(\S+)")
_NO_FALLTHROUGH = ("s_branch", "s_endpgm", "s_setpc_b64")


@dataclass
class Finding:
    line: int          # 1-based line of the vector memory instruction
    function: str
    writer: str        # the VALU instruction that wrote the SGPR
    states: int        # wait states between them on that path
    reader: str


def _sregs(text: str) -> set:
    out = set()
    for m in _SREG.finditer(text):
        if m.group(1) is not None:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
        else:
            out.add(int(m.group(3)))
    return out


def _operands(ins: str) -> list:
    parts = ins.split(None, 1)
    return [o.strip() for o in parts[1].split(",")] if len(parts) > 1 else []


def _valu_sgpr_writes(ins: str) -> set:
    if not ins.startswith("v_"):
        return set()
    ops = _operands(ins)
    out = _sregs(ops[0]) if ops else set()
    if ins.startswith(_SDST2) and len(ops) > 1:
        out |= _sregs(ops[1])
    return out


def _clean(line: str) -> str:
    return line.split(";")[0].strip()


def scan_text(text: str) -> list:
    raw = text.split("\n")
    lines = [_clean(l) for l in raw]
    labels = {}
    for k, l in enumerate(lines):
        if l.endswith(":") and " " not in l:
            labels[l[:-1]] = k
    branches_to = {}
    for k, l in enumerate(lines):
        m = _BRANCH.match(l)
        if m and m.group(1) in labels:
            branches_to.setdefault(m.group(1), []).append(k)
    func_of = []
    fn = ""
    for l in lines:
        if l.endswith(":") and not l.startswith("."):
            fn = l[:-1]
        func_of.append(fn)

    findings = []

    def is_label(l: str) -> bool:
        return l.endswith(":") and " " not in l

    def walk(j: int, used: set, states: int, seen: set, reader: int):
        # j: the instruction executed right before the point reached so far,
        # with `states` wait states counted from there to the reader
        after_label = False
        while j >= 0 and states < WAIT_STATES:
            l = lines[j]
            if is_label(l):
                if not l.startswith("."):
                    return  # function entry
                for b in branches_to.get(l[:-1], []):
                    if (b, states) not in seen:
                        seen.add((b, states))
                        walk(b, used, states, seen, reader)
                after_label = True
                j -= 1
                continue
            if not l or l.startswith("."):
                j -= 1
                continue
            if after_label and l.startswith(_NO_FALLTHROUGH):
                return  # the label is reached only by its branches
            after_label = False
            if _valu_sgpr_writes(l) & used:
                findings.append(Finding(reader + 1, func_of[reader], l, states, lines[reader]))
                return
            states += int(l.split()[1], 0) + 1 if l.startswith("s_nop") else 1
            j -= 1

    for k, l in enumerate(lines):
        if not l.startswith(_VMEM):
            continue
        used = set()
        for op in _operands(l):
            used |= _sregs(op)
        if used:
            walk(k - 1, used, 0, set(), k)
    return findings


def scan_file(path: str) -> list:
    with open(path) as f:
        return scan_text(f.read())


def main(argv) -> int:
    bad = 0
    for path in argv:
        for f in scan_file(path):
            bad += 1
            print(f"{path}:{f.line}: {f.function}: '{f.reader}' reads an SGPR {f.states} wait "
                  f"states after '{f.writer}' (needs {WAIT_STATES})")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
