"""CPU checks of the generated hand-scheduled loops read as text
(harp_amd/csrc/fwd_asm.inc, dq_asm.inc, dkdv_asm.inc) by tests/asm_check.py,
which shares no code with the generators or their scheduler:

* every register a loop writes is an output or a clobber of the kernel's asm
  statement (SGPRs, VGPRs, AGPRs, vcc, m0, scc), so the compiler keeps no
  value of its own in one across the loop;
* on every path through each loop, every dependent pair has the wait states
  of the gfx950 rules (MFMA -> VALU / DS / VMEM / MFMA srcA-B, VALU -> MFMA,
  v_exp -> VALU, VALU SGPR -> lane mask / SALU, m0 -> LDS-DMA, MFMA srcC ->
  overwrite), every LDS read is retired by an s_waitcnt lgkmcnt before its
  destination is used, and the loop leaves no hazard to the compiled code
  around it;
* planted mistakes fail: a dropped s_nop, an s_waitcnt moved one
  instruction later, a write to a register the statement does not declare.
"""

import pytest

from tests import asm_check as A

LOOPS = sorted(A.LOOPS)


@pytest.fixture(scope="module")
def loops():
    out = {}
    for n in LOOPS:
        inc, macro, _, _ = A.LOOPS[n]
        lines = A.macro_lines(inc, macro)
        out[n] = (lines, A.build(lines))
    return out


@pytest.mark.parametrize("name", LOOPS)
def test_written_registers_are_declared(name, loops):
    _, prog = loops[name]
    undeclared = A.written(prog) - A.declared(name)
    assert not undeclared, f"{name} loop writes {sorted(undeclared)} without declaring them"
    # the two the compiler could otherwise keep a value in
    assert {"m0", "scc"} <= A.declared(name)


@pytest.mark.parametrize("name", LOOPS)
def test_no_input_operand_is_written(name, loops):
    _, prog = loops[name]
    assert not [r for r in A.written(prog) if r.startswith("%")]


@pytest.mark.parametrize("name", LOOPS)
def test_wait_states_and_lds_waits(name, loops):
    _, prog = loops[name]
    bad = A.check(prog, strict=True)
    assert not bad, "\n".join(map(str, bad[:20]))


def test_parser_roles():
    i = A.parse_ins("v_mfma_f32_32x32x16_bf16 a[16:31], v[180:183], v[236:239], a[16:31]")
    assert i.kind == "mfma" and i.dst == [f"a{k}" for k in range(16, 32)] and i.srcC == i.dst
    assert i.src == [f"v{k}" for k in range(180, 184)] + [f"v{k}" for k in range(236, 240)]
    i = A.parse_ins("v_cndmask_b32_e32 v128, v128, v194, vcc")
    assert i.dst == ["v128"] and "vcc_lo" in i.mask
    i = A.parse_ins("buffer_load_dwordx4 v48, s[72:75], 0 offen lds")
    assert i.kind == "vmem" and "m0" in i.src and not i.dst
    i = A.parse_ins("s_addc_u32 s73, s73, 0")
    assert "scc" in i.src and "scc" in i.dst
    assert A.parse_ins("s_nop 12").states == 13
    assert A.parse_ins("s_waitcnt vmcnt(0) lgkmcnt(3)").lgkm == 3


@pytest.mark.parametrize("name", LOOPS)
def test_dropped_nop_fails(name, loops):
    lines, _ = loops[name]
    nops = [k for k, ln in enumerate(lines) if ln.startswith("s_nop")]
    # every s_nop in the loops is needed: dropping any of the first ones,
    # and the one before the statement's end, is caught
    for k in nops[:6] + nops[-1:]:
        bad = A.check(A.build(lines[:k] + lines[k + 1:]), strict=True)
        assert bad, f"dropping {lines[k]!r} at line {k} went unnoticed"


@pytest.mark.parametrize("name", LOOPS)
def test_late_lds_wait_fails(name, loops):
    lines, _ = loops[name]
    # an lgkmcnt wait directly before a vector instruction is there for that
    # instruction: issued one instruction later, the instruction reads or
    # overwrites an LDS result still in flight
    waits = [k for k, ln in enumerate(lines[:-1]) if ln.startswith("s_waitcnt lgkmcnt")
             and not (lines[k + 1].startswith("s_") or lines[k + 1].endswith(":"))]
    assert len(waits) > 50
    for k in waits[:8] + waits[-2:]:
        moved = lines[:k] + [lines[k + 1], lines[k]] + lines[k + 2:]
        bad = A.check(A.build(moved), strict=True)
        assert any(v.rule == "lgkmcnt" for v in bad), f"{lines[k]!r} moved past {lines[k + 1]!r} went unnoticed"


@pytest.mark.parametrize("name", LOOPS)
def test_undeclared_write_fails(name, loops):
    lines, _ = loops[name]
    k = next(k for k, ln in enumerate(lines) if ln.startswith("s_add_u32 m0"))
    planted = lines[:k] + ["s_mov_b32 s20, 0"] + lines[k:]
    assert "s20" in A.written(A.build(planted)) - A.declared(name)


def test_exit_hazard_fails():
    # an MFMA result read right after the statement without its wait states
    prog = A.build(["v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]", "s_nop 5"])
    assert any(v.rule == "exit_mfma" for v in A.check(prog))
    prog = A.build(["s_nop 1", "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]", "s_nop 12"])
    assert not A.check(prog)
    # entry: a VALU result of the code before the statement fed straight to an MFMA
    prog = A.build(["v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], 0", "s_nop 12"])
    assert any(v.rule == "valu_mfma" for v in A.check(prog))


def test_branch_joins_take_the_worst_path():
    # the fall-through path has the wait states, the branch path does not
    prog = A.build([
        "v_mfma_f32_32x32x16_bf16 v[16:31], v[0:3], v[4:7], 0",
        "s_cmp_eq_u32 s60, 0",
        "s_cbranch_scc1 .Lx_%=",
        "s_nop 12",
        ".Lx_%=:",
        "v_add_f32_e32 v40, v16, v17",
        "s_nop 0",
    ])
    bad = A.check(prog)
    assert any(v.rule == "mfma_raw" and v.have < 12 for v in bad)


def test_emitter_lds_waits_fit_the_counter():
    """The emitter's LDS waits never exceed the 4-bit lgkmcnt field: with 20
    reads outstanding, a wait that needs 18 left is emitted as 15 (retiring
    three more than needed), and the tracker keeps the 15 youngest."""
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "harp_amd" / "csrc"))
    import asm_sched
    em = asm_sched.Emitter()
    em.lds = [{f"v{i}"} for i in range(20)]
    em.wait_lgkm(18)
    assert em.lines[-1] == "s_waitcnt lgkmcnt(15)"
    assert em.lds == [{f"v{i}"} for i in range(5, 20)]
    em.wait_lgkm(0)
    assert em.lines[-1] == "s_waitcnt lgkmcnt(0)" and em.lds == []
