"""The build-time check of inline-asm loads (mindxsoup_amd/isa_check.py) on small listings in
the compiler's assembly format, each built so that one rule decides the outcome."""

import os

from mindxsoup_amd import isa_check

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def listing(body):
    return "\t.type\tk,@function\nk:\n" + body + "\n.Lfunc_end0:\n"


def asm_load(dst, op="global_load_dwordx2"):
    return f"\t;;#ASMSTART\n\t{op} {dst}, v1, s[4:5]\n\t;;#ASMEND\n"


def findings(body):
    return isa_check.check(listing(body)).get("k", [])


def test_use_after_covering_wait_is_clean():
    assert findings(asm_load("v[10:11]") + "\ts_waitcnt vmcnt(0)\n\tv_add_u32 v2, v10, v11\n"
                    "\ts_endpgm\n") == []


def test_use_before_wait_is_found():
    rep = findings(asm_load("v[10:11]") + "\tv_mov_b32 v2, v11\n\ts_endpgm\n")
    assert len(rep) == 1 and rep[0][2] == [11]


def test_write_to_pending_register_is_found():
    # the allocator reusing the register for another value while the load is in flight
    rep = findings(asm_load("v10", "global_load_dword") + "\tv_mov_b32 v10, 0\n\ts_endpgm\n")
    assert [r[2] for r in rep] == [[10]]


def test_vmcnt_retires_in_issue_order_and_counts_dma():
    # one younger instruction (a direct-to-LDS copy) after the load: vmcnt(1) retires it,
    # vmcnt(2) does not
    dma = "\t;;#ASMSTART\n\ts_mov_b32 m0, s2\n\tglobal_load_lds_dwordx4 v3, s[6:7]\n\t;;#ASMEND\n"
    ok = asm_load("v[10:11]") + dma + "\ts_waitcnt vmcnt(1)\n\tv_mov_b32 v2, v10\n\ts_endpgm\n"
    bad = asm_load("v[10:11]") + dma + "\ts_waitcnt vmcnt(2)\n\tv_mov_b32 v2, v10\n\ts_endpgm\n"
    assert findings(ok) == []
    assert len(findings(bad)) == 1


def test_compiler_visible_loads_count_but_are_not_tracked():
    # a load outside inline asm is the compiler's to wait for; it still ages the asm load
    body = (asm_load("v10", "global_load_dword") + "\tglobal_load_dword v20, v1, s[4:5]\n"
            "\ts_waitcnt vmcnt(1)\n\tv_mov_b32 v2, v10\n\ts_endpgm\n")
    assert findings(body) == []


def test_pending_on_one_path_of_a_merge_is_found():
    body = (asm_load("v10", "global_load_dword") +
            "\ts_cbranch_scc1 .LBB0_2\n"
            "\ts_waitcnt vmcnt(0)\n"
            ".LBB0_2:\n"
            "\tv_mov_b32 v2, v10\n"
            "\ts_endpgm\n")
    assert len(findings(body)) == 1
    # waiting on both paths is clean
    body_ok = body.replace(".LBB0_2:\n", ".LBB0_2:\n\ts_waitcnt vmcnt(0)\n")
    assert findings(body_ok) == []


def test_load_carried_around_a_loop_back_edge():
    # the load at the bottom of the loop is used at the top of the next iteration
    loop = (".LBB0_1:\n"
            "\tv_add_u32 v2, v2, v10\n" + asm_load("v10", "global_load_dword") +
            "\ts_cbranch_scc1 .LBB0_1\n"
            "\ts_waitcnt vmcnt(0)\n"
            "\ts_endpgm\n")
    # the read at the top, and the next load into the same register while the last one may
    # still be in flight
    assert [(k, regs) for k, _, regs in findings(loop)] == [(0, [10]), (1, [10])]
    fixed = loop.replace(".LBB0_1:\n", ".LBB0_1:\n\ts_waitcnt vmcnt(0)\n")
    assert findings(fixed) == []


def test_zeroed_mask_path_skips_the_flag_blocks_other_successor():
    # the compiler's join through a mask: coming from the loop (mask 0) vccz is taken, so the
    # moves below are reached only from the path that set -1 and has nothing in flight
    body = ("\ts_cbranch_scc1 .LBB0_3\n" + asm_load("v10", "global_load_dword") +
            "\ts_mov_b64 s[0:1], 0\n"
            "\ts_branch .LBB0_4\n"
            ".LBB0_3:\n"
            "\ts_mov_b64 s[0:1], -1\n"
            ".LBB0_4:\n"
            "\ts_and_b64 vcc, exec, s[0:1]\n"
            "\ts_cbranch_vccz .LBB0_6\n"
            "\tv_mov_b32 v10, v3\n"
            ".LBB0_6:\n"
            "\ts_waitcnt vmcnt(0)\n"
            "\ts_endpgm\n")
    assert findings(body) == []
    # with the masks swapped the load's path reaches the move
    swapped = body.replace("s_mov_b64 s[0:1], 0", "s_mov_b64 s[0:1], X").replace(
        "s_mov_b64 s[0:1], -1", "s_mov_b64 s[0:1], 0").replace("s_mov_b64 s[0:1], X",
                                                                "s_mov_b64 s[0:1], -1")
    assert [r[2] for r in findings(swapped)] == [[10]]
    # a different mask register decides nothing
    other = body.replace("s_and_b64 vcc, exec, s[0:1]", "s_and_b64 vcc, exec, s[2:3]")
    assert [r[2] for r in findings(other)] == [[10]]


def test_dead_path_after_endpgm_is_not_followed():
    body = (asm_load("v10", "global_load_dword") + "\ts_waitcnt vmcnt(0)\n\ts_endpgm\n")
    assert findings(body) == []


def test_built_gemm_assembly_is_clean():
    # the build writes the checked listing next to the objects; when present it stays clean
    path = os.path.join(ROOT, "mindxsoup_amd", "csrc", "_build", "nf4_gemm.s")
    if not os.path.exists(path):
        import pytest

        pytest.skip("library not built here")
    asm = open(path).read()
    assert "k_nf4_gemm_ws" in asm
    assert isa_check.check(asm) == {}
