"""CPU check of the compiled gfx950 device code: no vector memory instruction
reads an SGPR fewer than 5 wait states after a VALU instruction wrote it
(the hazard the library's inline-asm copies and loads must guard themselves;
tests/isa_check.py).  Compiles every library source to device assembly
with the build's flags (hipcc cross-compiles here, no GPU needed)."""
import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

from kan_amd import build as kbuild
import isa_check


def test_checker_finds_short_paths():
    hazard = """
k:
\tv_readfirstlane_b32 s2, v4
\ts_nop 2
\tglobal_load_dwordx4 v[0:3], v1, s[2:3]
\ts_endpgm
"""
    f = isa_check.scan_text(hazard)
    assert len(f) == 1 and f[0].states == 3 and "v_readfirstlane_b32 s2" in f[0].writer
    safe = hazard.replace("s_nop 2", "s_nop 4")
    assert isa_check.scan_text(safe) == []
    # an unrelated SGPR, and a carry-out write of the base
    assert isa_check.scan_text(hazard.replace("s2, v4", "s7, v4")) == []
    carry = "k:\n\tv_add_co_u32 v0, s[2:3], v1, v2\n\tglobal_load_dword v5, v1, s[2:3]\n"
    assert len(isa_check.scan_text(carry)) == 1


def test_checker_follows_branches():
    # the write sits before a branch to the label: 2 states on that path
    looped = """
k:
\ts_mov_b32 s4, 0
.LBB0_1:
\ts_nop 0
\tglobal_load_lds_dwordx4 v1, s[8:9]
\ts_add_i32 s4, s4, 1
\tv_readfirstlane_b32 s9, v7
\ts_cbranch_scc1 .LBB0_1
\ts_endpgm
"""
    f = isa_check.scan_text(looped)
    assert len(f) == 1 and f[0].states == 2
    # a label reached only by a branch from code with enough states: nothing
    far = """
k:
\tv_readfirstlane_b32 s9, v7
\ts_nop 4
\ts_branch .LBB0_2
\tv_readfirstlane_b32 s8, v6
\ts_endpgm
.LBB0_2:
\tglobal_load_lds_dwordx4 v1, s[8:9]
\ts_endpgm
"""
    assert isa_check.scan_text(far) == []


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc (ROCm) not installed")
def test_library_device_code_has_no_sgpr_vmem_hazard():
    hipcc = kbuild.hipcc()
    with tempfile.TemporaryDirectory() as td:
        def compile_one(src):
            out = os.path.join(td, os.path.splitext(src)[0] + ".s")
            cmd = [hipcc, *kbuild.COMMON_FLAGS, "--cuda-device-only", "-S", "-c",
                   os.path.join(kbuild.CSRC, src), "-o", out]
            r = subprocess.run(cmd, capture_output=True, text=True)
            assert r.returncode == 0, r.stderr[-2000:]
            return out
        with ThreadPoolExecutor(max_workers=len(kbuild.SOURCES)) as ex:
            outs = list(ex.map(compile_one, kbuild.SOURCES))
        findings = [(os.path.basename(o), f) for o in outs for f in isa_check.scan_file(o)]
    msg = "\n".join(f"{o}:{f.line} {f.function}: {f.reader} <- {f.writer} ({f.states} states)"
                    for o, f in findings[:20])
    assert not findings, msg
