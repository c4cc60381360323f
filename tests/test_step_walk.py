"""cusr_amd.benchmark.step_walk on a hand-written assembly fragment: the walk
follows the branches the instruction word's fields decide, counts each kind of
instruction on that path and stops at the next load of the word."""
from cusr_amd.benchmark import step_walk

ASM = """\
_Zkernel:
.LBB0_1:
\ts_load_dwordx2 s[12:13], s[0:1], 0x0
\ts_waitcnt lgkmcnt(0)
\ts_bfe_u32 s2, s12, 0x20007
\ts_cmp_eq_u32 s2, 2
\ts_cbranch_scc1 .LBB0_3
; %bb.2:
\tv_mov_b64_e32 v[0:1], v[2:3]
\ts_branch .LBB0_4
.LBB0_3:
\tds_read_b64 v[0:1], v4
\tv_mov_b64_e32 v[6:7], v[0:1]
.LBB0_4:
\ts_bitcmp1_b32 s13, 16
\ts_cbranch_scc0 .LBB0_6
; %bb.5:
\tv_mul_f64 v[8:9], v[8:9], v[0:1]
.LBB0_6:
\ts_add_i32 s20, s20, 1
\ts_cmp_lg_u32 s20, s21
\ts_cbranch_scc1 .LBB0_1
\ts_endpgm
_Znext:
"""


def test_walk_follows_the_word(tmp_path):
    p = tmp_path / "k.s"
    p.write_text(ASM)
    blocks, order = step_walk.parse(str(p), "_Zkernel")
    regs = {"s20": 0, "s21": 9}
    # operand kind CONST (bits 7..8 = 2) and scale_a (bit 48) set
    c, unknown = step_walk.walk(blocks, order, ".LBB0_1",
                                step_walk.word(1, ak=step_walk.CONST, sa=1), regs)
    assert not unknown
    assert (c["valu"], c["lds"], c["smem"]) == (2, 1, 1)
    assert c["branch"] == 3 and c["salu"] == 5
    # operand kind ACC, no scaling: the move, no LDS read, no multiply
    c, unknown = step_walk.walk(blocks, order, ".LBB0_1", step_walk.word(1), regs)
    assert not unknown
    assert (c["valu"], c["lds"], c["branch"]) == (1, 0, 4)
