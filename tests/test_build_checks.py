"""CPU tests of the build-time assembly check for inline-asm loads
(vllm-exact_amd/check_async_loads.py): it must reject a destination register touched before
the covering wait (straight line, through a branch, around a loop), a path that ends
uncovered, and compiler-generated M0 use, and accept the same code once a wait covers it."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
CHECK = ROOT / "vllm-exact_amd" / "check_async_loads.py"


def run(tmp_path, body):
    asm = tmp_path / "k.s"
    asm.write_text("_Zkernel:\n" + body + "\n.Lfunc_end0:\n")
    return subprocess.run([sys.executable, str(CHECK), str(asm), "_Zkernel"], capture_output=True, text=True)


LOAD = ";;#ASMSTART\nglobal_load_dwordx4 v[4:7], v[0:1], off\n;;#ASMEND\n"


def test_accepts_covered_load(tmp_path):
    r = run(tmp_path, LOAD + "global_load_dwordx4 v[8:11], v[2:3], off\ns_waitcnt vmcnt(1)\nv_mov_b32 v5, 0\ns_endpgm")
    assert r.returncode == 0, r.stdout


def test_rejects_touch_before_wait(tmp_path):
    r = run(tmp_path, LOAD + "v_mov_b32 v5, 0\ns_waitcnt vmcnt(0)\ns_endpgm")
    assert r.returncode == 1 and "v_mov_b32 v5" in r.stdout


def test_rejects_wait_that_does_not_cover(tmp_path):
    # vmcnt(1) with no younger memory operation leaves this load possibly in flight
    r = run(tmp_path, LOAD + "s_waitcnt vmcnt(1)\nv_add_u32_e32 v1, v6, v1\ns_waitcnt vmcnt(0)\ns_endpgm")
    assert r.returncode == 1


def test_rejects_touch_on_branch_path(tmp_path):
    body = (LOAD + "s_cbranch_scc1 .LBB0_2\ns_waitcnt vmcnt(0)\ns_branch .LBB0_3\n.LBB0_2:\nv_mov_b32 v7, 1\n"
            ".LBB0_3:\ns_waitcnt vmcnt(0)\ns_endpgm")
    r = run(tmp_path, body)
    assert r.returncode == 1 and "v_mov_b32 v7" in r.stdout


def test_rejects_uncovered_end_and_loop_reuse(tmp_path):
    assert run(tmp_path, LOAD + "s_endpgm").returncode == 1
    body = (".LBB0_1:\n" + LOAD + "v_mfma_i32_16x16x64_i8 a[0:3], v[4:7], v[4:7], a[0:3]\n"
            "s_cbranch_scc1 .LBB0_1\ns_waitcnt vmcnt(0)\ns_endpgm")
    assert run(tmp_path, body).returncode == 1


def test_rejects_compiler_m0_use(tmp_path):
    r = run(tmp_path, "s_mov_b32 m0, s2\n" + LOAD + "s_waitcnt vmcnt(0)\ns_endpgm")
    assert r.returncode == 1 and "m0" in r.stdout
