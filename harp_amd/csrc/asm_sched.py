"""Hazard-aware instruction emitter and gap-filling scheduler for the
hand-scheduled gfx950 loops (generated inline asm).

The emitter inserts the wait states that software must provide on gfx950.
Each rule is the count hipcc's own hazard recognizer uses for the same pair
in code it compiles, plus a margin where noted:
  MFMA (v_mfma_f32_32x32x16_bf16) vdst -> VALU / DS / VMEM read or write,
    or another MFMA's srcA / srcB                                 12 (13 used)
  MFMA vdst -> srcC of the same-shape MFMA on the same tuple        0
  VALU write -> MFMA read                                           1 (2 used)
  VALU write -> v_permlane32_swap read                              2
  transcendental (v_exp_f32) write -> VALU read                     1 (2 used)
  VALU write of an SGPR -> VALU lane-mask read or SALU read         2
  s_mov / s_add to m0 -> buffer_load ... lds                        1
  MFMA srcC read -> non-MFMA write of those registers              13 (margin)
LDS reads are tracked in issue order; an instruction touching a register an
outstanding LDS read writes first gets the s_waitcnt lgkmcnt(n) that retires
it (LDS operations complete in order).
"""
import re

MFMA_RAW = 13
REG_RE = re.compile(r"\b([vas])\[(\d+):(\d+)\]|\b([vas])(\d+)\b")


def regs_of(s):
    out = []
    for m in REG_RE.finditer(s):
        if m.group(1):
            k, a, b = m.group(1), int(m.group(2)), int(m.group(3))
            out += [f"{k}{i}" for i in range(a, b + 1)]
        else:
            out.append(f"{m.group(4)}{m.group(5)}")
    return out


def clobber_list(sgprs):
    """The asm statement's clobber list for a loop that writes the SGPRs
    `sgprs`: those, plus m0 (the LDS-DMA destination base) and scc (every
    compare, 32-bit add and branch condition), so the compiler keeps no
    value in either across the statement."""
    return ", ".join([f'"s{r}"' for r in sgprs] + ['"m0"', '"scc"'])


COST = {"mfma": 32, "valu": 4, "trans": 8, "perm": 8, "ds": 4, "vmem": 4, "salu": 1, "m0": 1}


class Ins:
    """One instruction.  kind: mfma valu trans perm ds vmem salu m0."""

    def __init__(self, text, kind, dst=(), src=(), srcC=()):
        self.text = text
        self.kind = kind
        self.dst = list(dst)
        self.src = list(src)
        self.srcC = list(srcC)
        self.cost = COST[kind]
        self.not_before = 0  # as a filler: only after this many MFMAs of the block


def ins(text, kind, dst="", src="", srcC=""):
    conv = lambda x: regs_of(x) if isinstance(x, str) else list(x)
    return Ins(text, kind, conv(dst), conv(src), conv(srcC))


class Emitter:
    """Linear instruction stream with hazard and LDS-wait tracking."""

    def __init__(self):
        self.lines = []
        self.pos = 0
        self.last_w = {}  # reg -> (position, kind, destination tuple)
        self.srcC_r = {}  # reg -> position of the last MFMA reading it as srcC
        self.lds = []     # outstanding LDS reads: destination register sets, oldest first

    @staticmethod
    def merged_entry(prevs):
        """Entry state after any of the blocks `prevs` (each measured from its
        own end): the most recent write of every register over all of them,
        and the longest outstanding-LDS list (they must agree in order)."""
        em = Emitter()
        for p in prevs:
            for r, (q, k, t) in p.last_w.items():
                q -= p.pos
                if r not in em.last_w or q > em.last_w[r][0]:
                    em.last_w[r] = (q, k, t)
            for r, q in p.srcC_r.items():
                q -= p.pos
                if r not in em.srcC_r or q > em.srcC_r[r]:
                    em.srcC_r[r] = q
            if len(p.lds) > len(em.lds):
                em.lds = [set(x) for x in p.lds]
        return em

    def ready_pos(self, i):
        need = self.pos
        dst_tuple = tuple(i.dst)
        for r in i.src + i.srcC:
            w = self.last_w.get(r)
            if not w:
                continue
            wp, wk, wt = w
            if wk == "mfma":
                if i.kind == "mfma" and r in i.srcC and wt == dst_tuple:
                    continue
                need = max(need, wp + MFMA_RAW + 1)
            elif wk in ("valu", "perm"):
                if r.startswith("s") or r == "vcc" or i.kind in ("mfma", "perm"):
                    need = max(need, wp + 3)
            elif wk == "trans":
                need = max(need, wp + 3)
            elif wk == "m0" and i.kind == "vmem":
                need = max(need, wp + 2)
        for r in i.dst:
            w = self.last_w.get(r)
            if w and w[1] == "mfma" and not (i.kind == "mfma" and w[2] == dst_tuple):
                need = max(need, w[0] + MFMA_RAW + 1)
            if i.kind != "mfma" and r in self.srcC_r:
                need = max(need, self.srcC_r[r] + MFMA_RAW + 1)
        return need

    def lgkm_needed(self, i):
        touch = set(i.src) | set(i.srcC) | set(i.dst)
        last = -1
        for k, s in enumerate(self.lds):
            if s & touch:
                last = k
        return None if last < 0 else len(self.lds) - 1 - last

    def raw(self, text, adv=0):
        """A line the tracker does not model (label, branch, waitcnt, SALU
        on registers no modelled instruction touches); adv = wait states it
        provides."""
        self.lines.append(text)
        self.pos += adv

    def nop(self, n):
        while n > 0:
            k = min(n, 16)
            self.raw(f"s_nop {k - 1}", k)
            n -= k

    def settle(self):
        """Pad so that every tracked MFMA result may be read."""
        far = max([p for (p, k, t) in self.last_w.values() if k == "mfma"] + [-100])
        if far + MFMA_RAW + 1 > self.pos:
            self.nop(far + MFMA_RAW + 1 - self.pos)

    def wait_lgkm(self, n):
        n = min(n, 15)  # the counter's field is 4 bits: waiting for 15 retires more, never fewer
        self.raw(f"s_waitcnt lgkmcnt({n})")
        self.lds = self.lds[len(self.lds) - n:] if n else []

    def emit(self, i):
        n = self.lgkm_needed(i)
        if n is not None:
            self.wait_lgkm(n)
        rp = self.ready_pos(i)
        if rp > self.pos:
            self.nop(rp - self.pos)
        self.lines.append(i.text)
        p = self.pos
        self.pos += 1
        t = tuple(i.dst)
        for r in i.dst:
            self.last_w[r] = (p, i.kind, t)
        if i.kind == "mfma":
            for r in i.srcC:
                self.srcC_r[r] = p
        if i.kind == "ds":
            self.lds.append(set(i.dst))
        return p

    def emit_all(self, seq):
        for i in seq:
            self.emit(i)


def fill_schedule(em, mfmas, fillers, budget=28, pinned=None, flush_war=False):
    """Issue `mfmas` in order.  Before MFMA k, the instructions pinned[k]
    (LDS prefetches, copies); after it, filler instructions in list order (a
    small lookahead may pass ones not yet hazard-ready, never one they depend
    on) for up to `budget` issue cycles, spread evenly over the gaps.
    flush_war: before MFMA k, if it writes registers that a pending filler
    allowed at k (not_before <= k) reads or writes, issue the allowed fillers
    up to the last such one, in list order: the MFMA must not overwrite what
    they still have to use.  (Fillers gated past k are work on the MFMA's
    result and stay pending.)
    Returns the fillers left over."""
    fillers = list(fillers)
    n = len(mfmas)
    for k, m in enumerate(mfmas):
        for p in (pinned or {}).get(k, []):
            em.emit(p)
        if flush_war and fillers:
            md = set(m.dst)
            last = -1
            for j, f in enumerate(fillers):
                if f.not_before <= k and md & (set(f.src) | set(f.dst) | set(f.srcC)):
                    last = j
            if last >= 0:
                keep = []
                for f in fillers[:last + 1]:
                    if f.not_before <= k:
                        em.emit(f)
                    else:
                        keep.append(f)
                fillers = keep + fillers[last + 1:]
        em.emit(m)
        left = sum(f.cost for f in fillers)
        target = min(budget, left / max(n - k, 1) + 2)
        spent = 0
        guard = 0
        while fillers and spent < target and guard < 64:
            guard += 1
            pick = None
            for j, f in enumerate(fillers[:10]):
                if f.not_before > k:
                    continue
                blocked = False
                for e in fillers[:j]:
                    if set(e.dst) & (set(f.src) | set(f.dst) | set(f.srcC)) or set(f.dst) & set(e.src):
                        blocked = True
                        break
                if blocked:
                    continue
                if em.ready_pos(f) <= em.pos and em.lgkm_needed(f) is None:
                    pick = j
                    break
            if pick is None:
                if spent == 0 and target >= budget and fillers[0].not_before <= k:
                    pick = 0
                else:
                    break
            f = fillers.pop(pick)
            em.emit(f)
            spent += f.cost
    return fillers
