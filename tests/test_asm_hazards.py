"""The generated gfx950 assembly holds no inline-asm load whose destination
registers are used before a wait covers the load (the fault class the
asm_check module describes). CPU only: compiles every source to device
assembly with the library's flags (a couple of minutes)."""
import importlib
import shutil
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _pkg():
    return importlib.import_module("tests.asm_check")


@pytest.mark.skipif(shutil.which("hipcc") is None and not Path("/opt/rocm/bin/hipcc").exists(),
                    reason="needs hipcc to generate the device assembly")
def test_no_inline_asm_load_hazards():
    ac = _pkg()
    res = ac.check_sources()
    assert res[""]["kernels"] > 300
    bad = {name: per for name, per in res.items() if name and per}
    assert not bad, bad


def test_checker_flags_a_register_copied_in_flight():
    """A planted case on the checker itself: the destination of an in-flight
    asm load copied before its wait is reported; after the wait it is not."""
    ac = _pkg()
    body = """
;;#ASMSTART
global_load_ushort v27, v[28:29], off
;;#ASMEND
;;#ASMSTART
global_load_dwordx4 v[2:5], v[6:7], off nt
;;#ASMEND
v_mov_b32_e32 v21, v27
s_endpgm
""".splitlines()
    f = ac.check_function(body)
    assert len(f) == 1 and "v_mov_b32_e32 v21, v27" in f[0][3]
    ok = body[:7] + ["s_waitcnt vmcnt(1)"] + body[7:]
    assert ac.check_function(ok) == []
    # the same copy reached only through a loop's back edge: the wait at the
    # top covers every load but the newest, which the copy reads
    loop = """
.LBB0_1:
s_waitcnt vmcnt(1)
v_mov_b32_e32 v21, v27
;;#ASMSTART
global_load_dwordx4 v[2:5], v[6:7], off nt
;;#ASMEND
;;#ASMSTART
global_load_ushort v27, v[28:29], off
;;#ASMEND
s_cbranch_scc0 .LBB0_1
s_endpgm
""".splitlines()
    f = ac.check_function(loop)
    assert len(f) == 1 and "v_mov_b32_e32 v21, v27" in f[0][3]
