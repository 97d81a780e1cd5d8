"""The MFMA hazard check (gfx950_gluon_tutorials_amd/isa_check.py) on small
hand-written listings: each planted hazard must be reported, and the same
listing with enough wait states must pass."""

from gfx950_gluon_tutorials_amd import isa_check


def _fn(body: str) -> str:
    return "k:\n" + body.strip("\n") + "\n\ts_endpgm\n"


MFMA32 = "\tv_mfma_f32_32x32x16_f16 a[0:15], v[0:3], v[4:7], a[0:15]\n"
MFMA_BF8 = "\tv_mfma_f32_32x32x64_f8f6f4 a[0:15], v[0:7], v[8:15], a[0:15] cbsz:1 blgp:1\n"


def test_read_after_mfma_needs_wait_states():
    bad = _fn(MFMA32 + "\ts_nop 3\n\tv_accvgpr_read_b32 v20, a15\n")
    good = _fn(MFMA32 + "\ts_nop 7\n\ts_nop 3\n\tv_accvgpr_read_b32 v20, a15\n")
    assert len(isa_check.check_text(bad)) == 1
    assert isa_check.check_text(good) == []


def test_bf8_32x32_needs_twenty():
    eighteen = _fn(MFMA_BF8 + "\ts_nop 7\n\ts_nop 7\n\ts_nop 1\n\tglobal_store_dwordx4 v[30:31], a[12:15], off\n")
    twenty = _fn(MFMA_BF8 + "\ts_nop 7\n\ts_nop 7\n\ts_nop 3\n\tglobal_store_dwordx4 v[30:31], a[12:15], off\n")
    assert len(isa_check.check_text(eighteen)) == 1
    assert isa_check.check_text(twenty) == []


def test_accumulating_chain_is_allowed_but_partial_source_is_not():
    chain = _fn(MFMA32 + MFMA32 + "\ts_nop 7\n\ts_nop 7\n\tv_accvgpr_read_b32 v20, a0\n")
    assert isa_check.check_text(chain) == []
    as_source = _fn(MFMA32 + "\tv_mfma_f32_32x32x16_f16 a[16:31], v[0:3], v[4:7], a[0:15]\n")
    assert len(isa_check.check_text(as_source)) == 1


def test_valu_write_then_mfma_read():
    bad = _fn("\tv_perm_b32 v2, v9, v8, v10\n" + MFMA32)
    good = _fn("\tv_perm_b32 v2, v9, v8, v10\n\ts_nop 1\n" + MFMA32)
    acc = _fn("\tv_accvgpr_write_b32 a3, v9\n" + MFMA32)
    assert len(isa_check.check_text(bad)) == 1
    assert isa_check.check_text(good) == []
    assert len(isa_check.check_text(acc)) == 1


def test_hazard_across_a_branch_and_a_back_edge():
    branch = _fn(MFMA32 + "\ts_cbranch_scc1 .LBB0_2\n\ts_nop 7\n\ts_nop 7\n.LBB0_2:\n\tv_accvgpr_read_b32 v20, a4\n")
    # Fall-through path has its wait states, the taken branch does not.
    assert len(isa_check.check_text(branch)) == 1
    loop = _fn(".LBB0_1:\n\tv_accvgpr_read_b32 v20, a4\n\ts_nop 7\n" + MFMA32 + "\ts_cbranch_scc1 .LBB0_1\n")
    assert len(isa_check.check_text(loop)) == 1
    loop_ok = _fn(".LBB0_1:\n\tv_accvgpr_read_b32 v20, a4\n\ts_nop 7\n" + MFMA32
                  + "\ts_nop 7\n\ts_nop 3\n\ts_cbranch_scc1 .LBB0_1\n")
    assert isa_check.check_text(loop_ok) == []


def test_unrelated_registers_and_comments_are_ignored():
    text = _fn(MFMA32 + "\tv_accvgpr_read_b32 v20, a16 ; reads a16, not a0..a15\n"
               "\t;;#ASMSTART\n\t;;#ASMEND\n\tv_add_u32_e32 v40, 0xa3, v41\n")
    assert isa_check.check_text(text) == []
