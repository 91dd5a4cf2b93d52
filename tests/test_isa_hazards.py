"""Every matrix-core result of the library's gfx950 build is touched only
after the required wait states, on every path (CPU: compiles to assembly).

The walk is checked first on hand-written listings with a planted short
distance, straight-line and across a branch join, so that a checker that
finds nothing is known to be able to find something."""

import os
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
