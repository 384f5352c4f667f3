"""CPU checks of the inline assembly in the library sources.

An asm statement that waits (s_waitcnt) on registers named as tied in/out
("+v") operands lets the compiler satisfy the tie by copying those registers
before the wait, which reads a load still in flight: the bf16 parity case
(1000, 100, 150, 6) once produced garbage rows that way.  No asm statement in
the sources may combine the two.
"""
import glob
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SOURCES = sorted(glob.glob(os.path.join(ROOT, "kan_amd", "csrc", "*.hip")) +
                 glob.glob(os.path.join(ROOT, "kan_amd", "csrc", "*.hpp")))


def asm_statements(text: str):
    """(line, body) of every asm(...) / asm volatile(...) statement, the body
    running to its balancing parenthesis."""
    out = []
    for m in re.finditer(r"\basm\s*(?:volatile\s*)?\(", text):
        depth, j = 1, m.end()
        while depth and j < len(text):
            depth += {"(": 1, ")": -1}.get(text[j], 0)
            j += 1
        out.append((text.count("\n", 0, m.start()) + 1, text[m.end():j - 1]))
    return out


def tied_vector_wait(body: str) -> bool:
    return "s_waitcnt" in body and re.search(r'"\+v"', body) is not None


def test_rule_detects_the_pattern():
    bad = 'asm volatile("s_waitcnt vmcnt(0)" : "+v"(a), "+v"(b));'
    ok_wait = 'asm volatile("s_waitcnt vmcnt(0)" ::: "memory");'
    ok_tied = 'asm volatile("v_mov_b32 %0, %0" : "+v"(a));'
    assert [tied_vector_wait(b) for _, b in asm_statements(bad)] == [True]
    assert [tied_vector_wait(b) for _, b in asm_statements(ok_wait + ok_tied)] == [False, False]


def test_sources_have_no_tied_operands_around_waits():
    assert SOURCES
    found = []
    for path in SOURCES:
        text = open(path).read()
        for line, body in asm_statements(text):
            if tied_vector_wait(body):
                found.append(f"{os.path.basename(path)}:{line}")
    assert not found, "inline asm waits on tied +v operands: " + ", ".join(found)
