"""Every matrix-core result of the library's gfx950 build is touched only
after the required wait states, on every path (CPU: compiles to assembly).

The walk is checked first on hand-written listings with a planted short
distance, straight-line and across a branch join, so that a checker that
finds nothing is known to be able to find something."""

import os
import re
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

import isa_hazards as H

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "loractl_amd", "csrc")
MFMA_SOURCES = ["lrq_gemm.hip", "lrq_gemm_mid.hip", "lrq_skinny.hip", "lrq_lora.hip"]

_HEAD = "\t.text\n\t.globl k\n\t.type k,@function\nk:\n"
_TAIL = "\ts_endpgm\n.Lfunc_end0:\n"


def _listing(body: str) -> list:
    return H.parse_asm(_HEAD + body + _TAIL)


def test_checker_flags_a_short_straight_line_distance():
    ks = _listing("\tv_mfma_f32_16x16x32_bf16 v[2:5], v[6:9], v[10:13], 0\n\ts_nop 6\n"
                  "\tv_add_f32_e32 v1, v5, v1\n")
    v, n = H.check_kernel(ks[0])
    assert n == 1 and len(v) == 1 and v[0].distance == 7 and v[0].required == 8


def test_checker_passes_the_required_distance():
    ks = _listing("\tv_mfma_f32_32x32x16_bf16 a[0:15], v[6:9], v[10:13], 0\n\ts_nop 7\n\ts_nop 3\n"
                  "\tv_accvgpr_read_b32 v1, a15\n")
    v, n = H.check_kernel(ks[0])
    assert n == 1 and not v


def test_checker_follows_a_branch_join():
    # the MFMA sits in a block that a uniform branch may skip; the read after
    # the join is 3 wait states behind it on the path through the block
    ks = _listing("\ts_cmp_lt_i32 s2, 17\n\ts_cbranch_scc1 .LBB0_2\n"
                  "\tv_mfma_f32_16x16x32_bf16 v[2:5], v[6:9], v[10:13], v[2:5]\n"
                  "\tv_mov_b32_e32 v20, 0\n"
                  ".LBB0_2:\n\ts_nop 1\n\tds_write_b32 v1, v5\n")
    v, n = H.check_kernel(ks[0])
    assert n == 1 and len(v) == 1 and v[0].distance == 3 and v[0].insn.startswith("ds_write_b32")


def test_checker_allows_a_chain_into_other_registers_but_not_a_partial_srcc():
    ks = _listing("\tv_mfma_f32_16x16x32_bf16 a[4:7], v[6:9], v[10:13], a[12:15]\n"
                  "\tv_mfma_f32_16x16x32_bf16 a[0:3], v[14:17], v[18:21], a[4:7]\n")
    v, n = H.check_kernel(ks[0])
    assert n == 2 and not v
    ks = _listing("\tv_mfma_f32_16x16x32_bf16 a[4:7], v[6:9], v[10:13], a[12:15]\n"
                  "\tv_mfma_f32_16x16x32_bf16 a[0:3], v[14:17], v[18:21], a[2:5]\n")
    v, n = H.check_kernel(ks[0])
    assert len(v) == 1 and v[0].distance == 0


def test_checker_allows_chained_accumulation():
    ks = _listing("\tv_mfma_f32_16x16x32_bf16 v[2:5], v[6:9], v[10:13], v[2:5]\n"
                  "\tv_mfma_f32_16x16x32_bf16 v[2:5], v[14:17], v[18:21], v[2:5]\n\ts_nop 7\n"
                  "\tv_add_f32_e32 v1, v5, v1\n")
    v, n = H.check_kernel(ks[0])
    assert n == 2 and not v


@pytest.fixture(scope="module")
def library_asm():
    with tempfile.TemporaryDirectory() as d:
        with ThreadPoolExecutor(len(MFMA_SOURCES)) as ex:
            texts = list(ex.map(lambda s: H.compile_asm(os.path.join(CSRC, s), os.path.join(ROOT, "include"), d),
                                MFMA_SOURCES))
    return dict(zip(MFMA_SOURCES, texts))


@pytest.mark.parametrize("src", MFMA_SOURCES)
def test_library_meets_mfma_wait_states(library_asm, src):
    total, bad = 0, []
    for k in H.parse_asm(library_asm[src]):
        v, n = H.check_kernel(k)
        total += n
        bad += v
    assert total > 0, f"no MFMA found in {src}"
    assert not bad, "\n".join(f"{x.kernel}: {x.mfma} -> {x.insn} after {x.distance} < {x.required}" for x in bad[:10])


# ---------------------------------------------------------------- counted waits
# The mid-size GEMM (k_mid) keeps MID_MST stages of loads in flight and, before
# each step's barrier, waits with a counted vmcnt for its own stage's copies
# into LDS. Such a count must not exceed MID_MST - 2 stages' worth of the
# loads a step issues: the compiler protects register results of loads with
# waits of its own, but not LDS written by buffer_load ... lds, so a count one
# too high lets a wavefront read a stage whose last copy is still in flight.
def _mid_mst() -> int:
    with open(os.path.join(CSRC, "lrq_kernels.h")) as f:
        m = re.search(r"constexpr int MID_MST = (\d+);", f.read())
    assert m, "MID_MST not found in lrq_kernels.h"
    return int(m.group(1))


def _bad_waits(pairs, mst):
    return [(w, n) for w, n in pairs if w is None or w > (mst - 2) * n]


def test_stage_wait_checker_flags_a_count_past_the_loads():
    ks = _listing(".LBB0_1:\n"
                  "\ts_waitcnt vmcnt(4)\n\ts_barrier\n"
                  "\tbuffer_load_dword v1, v0, s[0:3], 0 offen lds\n\tbuffer_load_dword v2, v0, s[0:3], 0 offen\n"
                  "\tv_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]\n"
                  "\ts_waitcnt vmcnt(3)\n\ts_barrier\n"
                  "\tbuffer_load_dword v3, v0, s[0:3], 0 offen\n"
                  "\tv_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]\n"
                  "\ts_cbranch_scc1 .LBB0_1\n")
    pairs = H.stage_waits(ks[0])
    assert pairs == [(4, 2), (3, 1)]
    assert _bad_waits(pairs, 4) == [(3, 1)]


def test_mid_gemm_waits_match_the_loads_per_stage(library_asm):
    mst = _mid_mst()
    seen = 0
    for k in H.parse_asm(library_asm["lrq_gemm_mid.hip"]):
        if "k_mid" not in k.name:
            continue
        pairs = H.stage_waits(k)
        assert pairs, f"{k.name}: no pipelined main loop found"
        assert not _bad_waits(pairs, mst), f"{k.name}: (vmcnt, loads per step) {pairs}"
        seen += 1
    assert seen > 0


# ---------------------------------------------------------------- DPP distances
_DPP = "\tv_mul_f32_dpp v1, v2, v1 row_newbcast:3 row_mask:0xf bank_mask:0xf bound_ctrl:1\n"


def test_dpp_checker_flags_a_valu_write_of_the_source():
    v, n = H.check_dpp(_listing("\tv_add_f32_e32 v2, v3, v4\n\ts_nop 0\n" + _DPP)[0])
    assert n == 1 and len(v) == 1 and v[0].required == H.DPP_AFTER_VALU


def test_dpp_checker_flags_an_exec_write_across_a_branch_join():
    ks = _listing("\ts_and_saveexec_b64 s[4:5], vcc\n\ts_cbranch_execz .LBB0_2\n\tv_mov_b32_e32 v9, 0\n"
                  ".LBB0_2:\n\ts_nop 1\n" + _DPP)
    v, n = H.check_dpp(ks[0])
    assert n == 1 and v and all(x.required == H.DPP_AFTER_EXEC for x in v)


def test_dpp_checker_passes_the_required_distances():
    v, n = H.check_dpp(_listing("\ts_mov_b64 exec, -1\n\tv_add_f32_e32 v2, v3, v4\n\ts_nop 3\n" + _DPP
                                + "\tv_add_f32_e32 v5, v1, v2\n" + _DPP.replace("v2,", "v6,"))[0])
    assert n == 2 and not v


@pytest.mark.parametrize("src", MFMA_SOURCES)
def test_library_meets_dpp_wait_states(library_asm, src):
    bad = []
    for k in H.parse_asm(library_asm[src]):
        v, _ = H.check_dpp(k)
        bad += v
    assert not bad, "\n".join(f"{x.kernel}: {x.insn} -> {x.mfma} after {x.distance} < {x.required}" for x in bad[:10])
