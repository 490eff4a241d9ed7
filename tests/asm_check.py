"""Static checker of the generated hand-scheduled loops (the .inc files that
harp_amd/csrc/fwd_asm_gen.py, dq_asm_gen.py and dkdv_asm_gen.py write), read
as text: it does not import the generators or share their bookkeeping.

Test infrastructure.  It parses the instruction strings of one loop macro,
builds the control-flow graph from its labels and branches, and runs a
forward data-flow analysis over every path (taking at each join the worst
case of the incoming paths) to check:

* wait states between dependent instructions, counted as the hardware and
  hipcc's hazard recognizer count them (one per instruction, n + 1 for
  `s_nop n`), against the gfx950 rules below;
* that every register an outstanding `ds_read*` writes is retired by an
  `s_waitcnt lgkmcnt(n)` before any instruction reads or writes it (LDS
  reads complete in issue order), and every SGPR an outstanding `s_load*`
  writes by `lgkmcnt(0)` (scalar loads may complete out of order);
* that the loop leaves no hazard to the compiled code after it (hipcc's
  hazard recognizer does not look into inline asm): at the end every MFMA
  result has its wait states and no LDS or scalar load is outstanding; and
  that the compiled code before it cannot hand it one: at the entry every
  register is taken as just written by a VALU instruction;
* which registers the loop writes (SGPRs, VGPRs, AGPRs, vcc, m0, scc), so a
  test can compare them with the asm statement's outputs and clobbers.

Wait-state rules (gfx950, v_mfma_f32_32x32x16_bf16 = 8 passes), as
`RULES[name] = (required, used by the generators)`; the check uses the
generators' counts unless asked for the hardware minimum:
  mfma_raw     MFMA vdst -> non-MFMA read or write, MFMA srcA/srcB   12 / 13
               (MFMA vdst -> srcC of an MFMA writing the same tuple: 0)
  valu_mfma    VALU write -> MFMA read                                1 / 2
  valu_perm    VALU write -> v_permlane32_swap read                   2 / 2
  trans_valu   v_exp_f32 write -> VALU read                           1 / 2
  valu_sgpr    VALU write of an SGPR (vcc) -> VALU lane-mask / SALU   2 / 2
  valu_vmem    VALU write of an SGPR -> VMEM read of it               5 / 5
  m0_lds       SALU write of m0 -> buffer_load ... lds                1 / 1
  mfma_war     MFMA srcC read -> non-MFMA write of those registers   11 / 13
"""
from __future__ import annotations

import re
from dataclasses import dataclass, field
from pathlib import Path
from typing import Dict, List, Optional, Set, Tuple

CSRC = Path(__file__).resolve().parents[1] / "harp_amd" / "csrc"

RULES = {
    "mfma_raw": (12, 13),
    "valu_mfma": (1, 2),
    "valu_perm": (2, 2),
    "trans_valu": (1, 2),
    "valu_sgpr": (2, 2),
    "valu_vmem": (5, 5),
    "m0_lds": (1, 1),
    "mfma_war": (11, 13),
}
CAP = 64  # distances beyond every rule are all alike

# SALU opcodes that write SCC, and those that read it
SCC_WRITERS = ("s_add_u32", "s_addc_u32", "s_sub_u32", "s_subb_u32", "s_add_i32", "s_sub_i32", "s_and_b32",
               "s_and_b64", "s_or_b32", "s_or_b64", "s_xor_b32", "s_xor_b64", "s_andn2_b32", "s_andn2_b64",
               "s_lshl_b32", "s_lshl_b64", "s_lshr_b32", "s_lshr_b64", "s_ashr_i32", "s_bfe_u32", "s_bfe_i32",
               "s_max_i32", "s_max_u32", "s_min_i32", "s_min_u32", "s_not_b32", "s_abs_i32")
SCC_READERS = ("s_addc_u32", "s_subb_u32", "s_cbranch_scc0", "s_cbranch_scc1", "s_cselect_b32", "s_cselect_b64")

_REG = re.compile(r"^-?\|?([vas])\[(\d+):(\d+)\]\|?$|^-?\|?([vas])(\d+)\|?$")


def regs(tok: str) -> List[str]:
    """Register names of one operand token ('v[4:7]' -> v4..v7; 'vcc' ->
    vcc_lo, vcc_hi; '%[c2]' -> '%c2'); literals give []."""
    tok = tok.strip()
    if tok.startswith("%["):
        return ["%" + tok[2:-1]]
    if tok in ("vcc", "exec"):
        return [tok + "_lo", tok + "_hi"]
    if tok in ("m0", "scc", "vcc_lo", "vcc_hi"):
        return [tok]
    m = _REG.match(tok)
    if not m:
        return []
    if m.group(1):
        k, a, b = m.group(1), int(m.group(2)), int(m.group(3))
        return [f"{k}{i}" for i in range(a, b + 1)]
    return [f"{m.group(4)}{m.group(5)}"]


@dataclass
class Ins:
    text: str
    op: str
    kind: str                      # mfma valu trans perm ds vmem smem salu branch wait nop barrier
    dst: List[str] = field(default_factory=list)
    src: List[str] = field(default_factory=list)
    srcC: List[str] = field(default_factory=list)
    mask: List[str] = field(default_factory=list)   # SGPRs read as a lane mask (VALU) or by SALU
    target: Optional[str] = None
    cond: bool = False
    lgkm: Optional[int] = None
    vm: Optional[int] = None
    states: int = 1                # wait states the instruction provides


def _operands(rest: str) -> List[str]:
    rest = re.sub(r"\b(offset|offset0|offset1):\S+", "", rest)
    rest = re.sub(r"\b(offen|lds|clamp|glc|slc|nt|sc0|sc1|idxen|off)\b", "", rest)
    return [t.strip() for t in rest.split(",") if t.strip()]


def parse_ins(line: str) -> Ins:
    """One instruction string -> Ins with its operand roles."""
    op, _, rest = line.strip().partition(" ")
    ops = _operands(rest)
    r = [regs(t) for t in ops]
    if op.startswith("v_mfma"):
        return Ins(line, op, "mfma", dst=r[0], src=r[1] + r[2], srcC=r[3])
    if op.startswith("ds_read"):
        return Ins(line, op, "ds", dst=r[0], src=r[1])
    if op.startswith("ds_write"):
        return Ins(line, op, "ds", src=sum(r, []))
    if op.startswith("buffer_load") and " lds" in " " + rest:
        return Ins(line, op, "vmem", src=sum(r, []) + ["m0"])
    if (op.startswith("buffer_") or op.startswith("global_")) and "load" in op:
        # a load into registers would need vmcnt tracking, which the loops
        # have no use for: refuse rather than pass it unchecked
        raise ValueError(f"vector memory load into registers is not modelled: {line!r}")
    if op.startswith("buffer_store") or op.startswith("global_store"):
        return Ins(line, op, "vmem", src=sum(r, []))
    if op.startswith("s_load") or op.startswith("s_buffer_load"):
        return Ins(line, op, "smem", dst=r[0], src=sum(r[1:], []))
    if op == "s_nop":
        return Ins(line, op, "nop", states=int(ops[0], 0) + 1)
    if op == "s_waitcnt":
        i = Ins(line, op, "wait")
        m = re.search(r"lgkmcnt\((\d+)\)", rest)
        i.lgkm = int(m.group(1)) if m else None
        m = re.search(r"vmcnt\((\d+)\)", rest)
        i.vm = int(m.group(1)) if m else None
        return i
    if op == "s_barrier":
        return Ins(line, op, "barrier")
    if op in ("s_branch", "s_cbranch_scc0", "s_cbranch_scc1"):
        i = Ins(line, op, "branch", target=ops[0], cond=op != "s_branch")
        if i.cond:
            i.src = ["scc"]
        return i
    if op.startswith("s_"):
        if op.startswith("s_cmp"):
            i = Ins(line, op, "salu", dst=["scc"], src=sum(r, []))
        else:
            i = Ins(line, op, "salu", dst=r[0] + (["scc"] if op in SCC_WRITERS else []), src=sum(r[1:], []))
        if op in SCC_READERS:
            i.src.append("scc")
        i.mask = [x for x in i.src if x.startswith("vcc") or x.startswith("s")]
        return i
    if op.startswith("v_"):
        kind = "trans" if op.startswith("v_exp") else ("perm" if op.startswith("v_permlane") else "valu")
        if op.startswith("v_permlane"):
            return Ins(line, op, kind, dst=r[0] + r[1], src=r[0] + r[1])
        dst, src = r[0], sum(r[1:], [])
        mask = []
        if op.startswith("v_cndmask") or op.startswith("v_addc") or op.startswith("v_subb"):
            vm = [x for x in src if x.startswith("vcc") or re.match(r"s\d", x)]
            mask = vm
            if op.endswith("_e32") and not vm:
                src = src + ["vcc_lo", "vcc_hi"]
                mask = ["vcc_lo", "vcc_hi"]
        if op.startswith("v_cmp") and op.endswith("_e32"):
            dst = ["vcc_lo", "vcc_hi"]
            src = sum(r[1:], []) if len(r) > 2 else sum(r, [])
        return Ins(line, op, kind, dst=dst, src=src, mask=mask)
    raise ValueError(f"instruction the checker does not know: {line!r}")


def macro_lines(inc: Path, macro: str) -> List[str]:
    """The instruction strings (and labels) of one #define in a generated
    .inc file, in order."""
    txt = inc.read_text()
    m = re.search(r"#define " + re.escape(macro) + r" \\\n((?:.*\\\n)*.*)", txt)
    if not m:
        raise KeyError(macro)
    out = []
    for s in re.findall(r'"((?:[^"\\]|\\.)*)"', m.group(1)):
        for part in s.replace("\\n", "\n").replace("\\t", "").split("\n"):
            part = part.strip()
            if part:
                out.append(part)
    return out


def clobber_list(inc: Path, macro: str) -> List[str]:
    txt = inc.read_text()
    m = re.search(r"#define " + re.escape(macro) + r" (.*)", txt)
    return re.findall(r'"([^"]+)"', m.group(1))


@dataclass
class Program:
    ins: List[Ins]
    labels: Dict[str, int]          # label -> index of the next instruction


def build(lines: List[str]) -> Program:
    ins, labels = [], {}
    for ln in lines:
        if ln.endswith(":"):
            labels[ln[:-1]] = len(ins)
        else:
            ins.append(parse_ins(ln))
    for i in ins:
        if i.kind == "branch" and i.target not in labels:
            raise ValueError(f"branch to an unknown label: {i.text}")
    return Program(ins, labels)


def written(p: Program) -> Set[str]:
    out = set()
    for i in p.ins:
        out |= set(i.dst)
    return out


# ---------------------------------------------------------------- data flow
#
# The analysis runs per basic block.  At a block's entry the state is, per
# register, the wait states since its last write of each kind (the minimum
# over the paths into the block), the wait states since an MFMA last read it
# as srcC, and for each register an outstanding ds_read writes the fewest LDS
# reads issued after that one; plus the SGPRs an outstanding s_load writes.
# Inside a block a local clock (wait states issued so far) turns those into
# times, so an instruction costs work only for the registers it touches.

Entry = Tuple[Dict[str, Dict[Tuple[str, Tuple[str, ...]], int]], Dict[str, int], Dict[str, int], frozenset]


@dataclass
class Violation:
    index: int
    text: str
    rule: str
    have: int
    need: int

    def __str__(self):
        return f"#{self.index} {self.text!r}: {self.rule} has {self.have} wait states, needs {self.need}"


def _need(rule: str, strict: bool) -> int:
    return RULES[rule][1] if strict else RULES[rule][0]


def _rule_for(kind: str, r: str, i: Ins) -> Optional[str]:
    """The rule a read of register r (last written by an instruction of
    `kind`, not an MFMA) by instruction i falls under, if any."""
    if kind in ("valu", "trans", "perm"):
        if i.kind == "mfma":
            return "valu_mfma"
        if i.kind == "perm":
            return "valu_perm"
        if kind == "trans" and i.kind in ("valu", "trans"):
            return "trans_valu"
        if r.startswith("s") or r.startswith("vcc"):
            if i.kind in ("valu", "trans", "perm"):
                return "valu_sgpr" if r in i.mask else None
            if i.kind == "salu":
                return "valu_sgpr"
            if i.kind == "vmem":
                return "valu_vmem"
        return None
    if kind == "salu" and r == "m0" and i.kind == "vmem":
        return "m0_lds"
    return None


def _blocks(p: Program):
    """Basic blocks as (start, end) index ranges, and each block's successors."""
    n = len(p.ins)
    starts = {0} | set(p.labels.values())
    for k, i in enumerate(p.ins):
        if i.kind == "branch":
            starts.add(k + 1)
    starts = sorted(x for x in starts if x <= n)
    blocks = {}
    for j, st in enumerate(starts):
        en = starts[j + 1] if j + 1 < len(starts) else n
        if st == n:
            blocks[st] = (st, st, [])
            continue
        last = p.ins[en - 1]
        if last.kind == "branch":
            t = p.labels[last.target]
            succ = [t, en] if last.cond else [t]
        else:
            succ = [en]
        blocks[st] = (st, en, succ)
    if n not in blocks:
        blocks[n] = (n, n, [])
    return blocks


def _run_block(p: Program, st: int, en: int, entry: Entry, strict: bool, found: Dict) -> Entry:
    w0, c0, lds0, sm = entry
    # local representation: write end-times (dist = clock - t), LDS issue indices
    wt: Dict[str, Dict[Tuple[str, Tuple[str, ...]], int]] = {r: {k: -d for k, d in dd.items()} for r, dd in w0.items()}
    ct = {r: -d for r, d in c0.items()}
    lidx = {r: -a - 1 for r, a in lds0.items()}
    clock = 0
    nds = 0
    for k in range(st, en):
        i = p.ins[k]
        reads = i.src + i.srcC
        touched = set(reads) | set(i.dst)
        for r in touched:
            for (kind, tup), t in wt.get(r, {}).items():
                dist = min(CAP, clock - t)
                if kind == "mfma":
                    if i.kind == "mfma":
                        same = tuple(i.dst) == tup
                        if same and (r in i.srcC or (r in i.dst and r not in i.src)):
                            continue
                    rule = "mfma_raw"
                elif r in reads:
                    rule = _rule_for(kind, r, i)
                else:
                    rule = None
                if rule and dist < _need(rule, strict):
                    v = found.get((k, rule))
                    if v is None or dist < v.have:
                        found[(k, rule)] = Violation(k, i.text, rule, dist, _need(rule, strict))
            if r in lidx:
                found.setdefault((k, "lgkmcnt"), Violation(k, i.text, "lgkmcnt", nds - lidx[r] - 1, -1))
            if r in sm:
                found.setdefault((k, "smem_lgkmcnt"), Violation(k, i.text, "smem_lgkmcnt", 0, -1))
        if i.kind != "mfma":
            for r in i.dst:
                if r in ct and clock - ct[r] < _need("mfma_war", strict):
                    found.setdefault((k, "mfma_war"), Violation(k, i.text, "mfma_war", clock - ct[r],
                                                                _need("mfma_war", strict)))
        # effects
        if i.kind == "wait" and i.lgkm is not None:
            n = i.lgkm
            lidx = {r: x for r, x in lidx.items() if nds - x - 1 < n}
            if n == 0:
                sm = frozenset()
        if i.kind == "ds":
            for r in i.dst:
                lidx[r] = nds
            nds += 1
        if i.kind == "smem":
            sm = sm | frozenset(i.dst)
        clock += i.states
        if i.kind in ("mfma", "valu", "trans", "perm", "salu", "smem", "ds", "vmem"):
            tup = tuple(i.dst)
            for r in i.dst:
                wt[r] = {(i.kind, tup): clock}
        if i.kind == "mfma":
            for r in i.srcC:
                ct[r] = clock
    w = {r: {key: min(CAP, clock - t) for key, t in dd.items()} for r, dd in wt.items()}
    c = {r: min(CAP, clock - t) for r, t in ct.items()}
    lds = {r: min(CAP, nds - x - 1) for r, x in lidx.items()}
    return (w, c, lds, sm)


def _merge(a: Entry, b: Entry) -> Entry:
    w = {r: dict(d) for r, d in a[0].items()}
    for r, d in b[0].items():
        t = w.setdefault(r, {})
        for key, v in d.items():
            t[key] = min(t.get(key, CAP), v)
    c = dict(a[1])
    for r, v in b[1].items():
        c[r] = min(c.get(r, CAP), v)
    lds = dict(a[2])
    for r, v in b[2].items():
        lds[r] = min(lds.get(r, CAP), v)
    return (w, c, lds, a[3] | b[3])


def entry_state(p: Program) -> Entry:
    """Every register the loop touches taken as written by a VALU
    instruction just before the statement (the compiled code before it)."""
    w = {}
    for i in p.ins:
        for r in i.src + i.srcC + i.dst:
            if (r[0] in "vas" and r[1:].isdigit()) or r.startswith("vcc"):
                w[r] = {("valu", (r,)): 0}
    return (w, {}, {}, frozenset())


def check(p: Program, strict: bool = True) -> List[Violation]:
    """Data-flow check of every path through the loop; returns the
    violations (an empty list when the loop is clean)."""
    n = len(p.ins)
    blocks = _blocks(p)
    at: Dict[int, Entry] = {0: entry_state(p)}
    work = [0]
    found: Dict[Tuple[int, str], Violation] = {}
    while work:
        st = work.pop()
        b0, b1, succ = blocks[st]
        out = _run_block(p, b0, b1, at[st], strict, found)
        for t in succ:
            if t not in at:
                at[t] = out
                work.append(t)
            else:
                merged = _merge(at[t], out)
                if merged != at[t]:
                    at[t] = merged
                    work.append(t)
    # the end of the statement: the compiled code after it sees no hazard
    end = at.get(n)
    if end is not None:
        w, c, lds, sm = end
        worst = min([d for dd in w.values() for (kind, _), d in dd.items() if kind == "mfma"] + [CAP])
        if worst < _need("mfma_raw", strict):
            found[(n, "exit_mfma")] = Violation(n, "<end of statement>", "exit_mfma", worst, _need("mfma_raw", strict))
        if lds:
            found[(n, "exit_lgkmcnt")] = Violation(n, "<end of statement>", "exit_lgkmcnt", len(lds), 0)
        if sm:
            found[(n, "exit_smem")] = Violation(n, "<end of statement>", "exit_smem", len(sm), 0)
        worst_c = min(list(c.values()) + [CAP])
        if worst_c < _need("mfma_war", strict):
            found[(n, "exit_mfma_war")] = Violation(n, "<end of statement>", "exit_mfma_war", worst_c,
                                                    _need("mfma_war", strict))
    return sorted(found.values(), key=lambda v: v.index)


LOOPS = {
    "fwd": (CSRC / "fwd_asm.inc", "HARP_FWD_ASM_LOOP", "HARP_FWD_ASM_SGPR_CLOBBERS", CSRC / "fwd_asm.hip"),
    "dq": (CSRC / "dq_asm.inc", "HARP_DQ_ASM_LOOP", "HARP_DQ_ASM_SGPR_CLOBBERS", CSRC / "dq_asm.hip"),
    "dkdv": (CSRC / "dkdv_asm.inc", "HARP_DKDV_ASM_LOOP", "HARP_DKDV_ASM_SGPR_CLOBBERS", CSRC / "dkdv_asm.hip"),
}


def loop_program(name: str, lines: Optional[List[str]] = None) -> Program:
    inc, macro, _, _ = LOOPS[name]
    return build(lines if lines is not None else macro_lines(inc, macro))


def declared(name: str) -> Set[str]:
    """Registers the kernel's asm statement names as outputs ("{v[a:b]}" /
    "{a[a:b]}" constraints) or clobbers (the generated SGPR list and the
    literal clobbers in the .hip file)."""
    inc, macro, clob, hip = LOOPS[name]
    src = hip.read_text()
    start = src.index(f"asm volatile({macro}")
    end = src.index(");", start)
    stmt = src[start:end]
    out = set()
    for k, a, b in re.findall(r'"\+?=?\{([va])\[(\d+):(\d+)\]\}"', stmt):
        out |= {f"{k}{i}" for i in range(int(a), int(b) + 1)}
    lits = re.findall(r'"(memory|vcc|m0|scc|exec)"', stmt)
    for x in lits:
        out |= set(regs(x)) if x in ("vcc", "exec") else {x}
    for r in clobber_list(inc, clob):
        out |= set(regs(r))
    return out
