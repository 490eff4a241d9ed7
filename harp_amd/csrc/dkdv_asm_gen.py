"""Generator of the hand-scheduled main loop of dkdv_asm_kernel
(dkdv_asm.hip), written to dkdv_asm.inc as one inline-asm string
(HARP_DKDV_ASM_LOOP).

Run by harp_amd/build.py before compiling; `python dkdv_asm_gen.py` rewrites
the file by hand.

Work split: a block of 4 waves x 64 keys (one wave per SIMD), D = 128.  A
wave's keys form two 32-key groups kg; every Q, dO, Q^T or dO^T fragment read
from LDS feeds one MFMA per group.  dK (kg, 32-wide d block db) accumulates
in a[64 kg + 16 db], dV in a[128 + 64 kg + 16 db] (fp32, row = key, lane =
d); the wave's K rows are the B operands of S = Q K^T in v32..v95; its V rows
(the B operands of dP = dO V^T) are read from the block's padded V tile in
LDS.  Queries stream in 32-query blocks J through five 16 KiB LDS buffers (Q
rows at +0, dO rows at +8 KiB), copied three blocks ahead, with a barrier
before every slot; the per-query statistics (-LSE / scale and -D, two fp32
planes) are copied beside them into a per-wave area and read back as the
initial values of the S and dP accumulators (C row = query: 16 B broadcast
reads), so the softmax needs no per-row operand.

Slot J (one per query block):
  MFMAs  phase 1: dV += P^T(J-1) dO(J-1), dK += dS^T(J-1) Q(J-1)  (32;
                  P / dS bf16 as A operands straight from the accumulator
                  layout, dO^T / Q^T by transposed LDS reads)
         phase 2: S(J+1) = Q K^T - LSE/scale, dP(J+1) = dO V^T - D  (32)
  VALU   dS = P dP of block J, P and dS rounded to bf16 once the phase-1
         MFMAs that read the previous block's have issued; P = exp2(S c) of
         block J + 1 after its S MFMAs (clamped to [0, 1])
  copies of block J + 3 (Q, dO rows and the statistics rows)
The read address registers point at a base buffer and the offsets select the
buffer (ds_read offsets reach 64 KiB: four of the five buffers from a base);
they move between base buffers 0 and 1 twice per trip around the buffers.
Query rows past T load as zero with zero statistics: their P is 1 but their
dO and Q rows are zero, so they add nothing.  Pad keys (past the chunk's
valid length) get zero dK / dV in the kernel's epilogue.
The reference math is ring_attn.cpp:2577-2829 (ring_attention_backward:
dV = P^T dO, dK = dS^T Q scaled), as dkdv_kernel in ra_kernels.hip computes
it.
"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from asm_sched import Emitter, clobber_list, fill_schedule, ins  # noqa: E402
from fwd_asm_gen import a, lbl, s, v  # noqa: E402

# ---- registers ------------------------------------------------------------
RADDR, TADDR = 0, 8           # Q / dO row-read and transposed-read addresses
VADDR, STADDR = 16, 17        # the wave's V rows; its statistics area
DOFFQ, DOFFG, SOFF = 18, 20, 22   # copy offsets (Q rows, dO rows, statistics)
KB = 32                       # K^T B operands: kg * 32 + ks * 4
S, DP = 96, 128               # S, dP accumulators: kg * 16 + r
PB, DSB = 160, 176            # P, dS bf16: kg * 8 + h2 * 4 + w
INS, INP = 192, 208           # initial S / dP accumulator values (both groups)
T_RING = (224, 228, 232, 236)           # dO^T / Q^T fragments (phase 1)
A_RING = (240, 244, 248)                # Q / dO row fragments (phase 2)
V_RING = (252, 24, 28, 232, 236)        # V row fragments (phase 2)
# SGPRs: buffer descriptors of the Q rows, dO rows and the two statistics
# planes (word 0-1 base, word 2 bytes left), the block counter
DQ, DG, DS0, DS1, J = 60, 64, 68, 72, 76
SGPR_CLOBBER = list(range(60, 77))

NBUF = 5
BUF = 16384                   # bytes per buffer: Q rows (8 KiB), dO rows (8 KiB)
QOFF, GOFF = 0, 8192
VROW = 272                    # padded V row
VKG = 32 * VROW               # 32 rows: one key group
ST_BUF = 512                  # statistics per wave and buffer: plane 0, plane 1 (256 B each)
AHEAD = 3                     # copies run this many blocks ahead
BUDGET = 20


def dk_acc(kg, db):
    return a(64 * kg + 16 * db, 16)


def dv_acc(kg, db):
    return a(128 + 64 * kg + 16 * db, 16)


def mf(acc, fa, fb, c):
    return ins(f"v_mfma_f32_32x32x16_bf16 {acc}, {fa}, {fb}, {c}", "mfma", dst=acc, src=f"{fa} {fb}",
               srcC=(c if c.startswith(("v[", "a[")) else ""))


# phase 1 pairs n = 0..15: even n dV (idx = n // 2), odd n dK; idx -> h2 = idx // 4, db = idx % 4
def p1_pair(n):
    idx = n // 2
    h2, db = idx // 4, idx % 4
    fr = v(T_RING[n % 4], 4)
    out = []
    for kg in range(2):
        if n % 2 == 0:
            acc, fa = dv_acc(kg, db), v(PB + kg * 8 + h2 * 4, 4)
        else:
            acc, fa = dk_acc(kg, db), v(DSB + kg * 8 + h2 * 4, 4)
        out.append(mf(acc, fa, fr, acc))
    return out


def t_read(n, rel):
    """transposed fragment of pair n: dO^T (even n) or Q^T (odd n), queries
    16 h2 .., d block db, from the buffer rel above the one TADDR points at"""
    idx = n // 2
    h2, db = idx // 4, idx % 4
    f = T_RING[n % 4]
    off = rel * BUF + (GOFF if n % 2 == 0 else QOFF) + h2 * 4096
    assert 0 <= off < 65536
    return [ins(f"ds_read_b64_tr_b16 {v(f, 2)}, {v(TADDR + db)} offset:{off}", "ds", dst=v(f, 2), src=v(TADDR + db)),
            ins(f"ds_read_b64_tr_b16 {v(f + 2, 2)}, {v(TADDR + 4 + db)} offset:{off}", "ds", dst=v(f + 2, 2),
                src=v(TADDR + 4 + db))]


# phase 2 pairs m = 0..15: m < 8 S(ks = m), m >= 8 dP(ks = m - 8)
def p2_pair(m):
    out = []
    fa = v(A_RING[m % 3], 4)
    if m < 8:
        ks = m
        for kg in range(2):
            acc = v(S + 16 * kg, 16)
            out.append(mf(acc, fa, v(KB + kg * 32 + ks * 4, 4), v(INS, 16) if ks == 0 else acc))
    else:
        ks = m - 8
        for kg in range(2):
            acc = v(DP + 16 * kg, 16)
            out.append(mf(acc, fa, v(V_RING[(2 * ks + kg) % 5], 4), v(INP, 16) if ks == 0 else acc))
    return out


def a_read(m, rel):
    """row fragment of phase-2 pair m from the buffer rel above the one RADDR points at"""
    ks = m % 8
    f = A_RING[m % 3]
    off = rel * BUF + (QOFF if m < 8 else GOFF)
    assert 0 <= off < 65536
    return [ins(f"ds_read_b128 {v(f, 4)}, {v(RADDR + ks)} offset:{off}", "ds", dst=v(f, 4), src=v(RADDR + ks))]


def v_reads(ks):
    out = []
    for kg in range(2):
        f = V_RING[(2 * ks + kg) % 5]
        out.append(ins(f"ds_read_b128 {v(f, 4)}, {v(VADDR)} offset:{kg * VKG + ks * 32}", "ds", dst=v(f, 4),
                       src=v(VADDR)))
    return out


def init_reads(buf):
    """initial S / dP accumulators of a block: register 4 j + i of lane half g
    holds query row 8 j + 4 g + i (STADDR carries 16 g)"""
    out = []
    for plane, base in ((0, INS), (1, INP)):
        for j in range(4):
            off = buf * ST_BUF + plane * 256 + j * 32
            out.append(ins(f"ds_read_b128 {v(base + 4 * j, 4)}, {v(STADDR)} offset:{off}", "ds",
                           dst=v(base + 4 * j, 4), src=v(STADDR)))
    return out


def dma(i, buf):
    """copy instruction i of a block into buffer buf: 0, 1 Q rows; 2, 3 dO
    rows; 4, 5 the statistics planes"""
    if i < 4:
        t, half = i // 2, i % 2
        base = buf * BUF + (GOFF if t else QOFF) + half * 1024
        desc, off = (s(DG, 4), v(DOFFG + half)) if t else (s(DQ, 4), v(DOFFQ + half))
        return [ins(f"s_add_u32 m0, %[dbase], {base}", "m0", dst=["m0"]),
                ins(f"buffer_load_dwordx4 {off}, {desc}, 0 offen lds", "vmem", src=[off, "m0"])]
    plane = i - 4
    base = buf * ST_BUF + plane * 256
    desc = s(DS0 if plane == 0 else DS1, 4)
    return [ins(f"s_add_u32 m0, %[sbase], {base}", "m0", dst=["m0"]),
            ins(f"buffer_load_dword {v(SOFF)}, {desc}, 0 offen lds", "vmem", src=[v(SOFF), "m0"])]


def desc_advance():
    """the four descriptors to the next query block (bytes left clamped at 0)"""
    out = []
    for d, step in ((DQ, "%[qstep]"), (DG, "%[gstep]"), (DS0, "128"), (DS1, "128")):
        out += [f"s_add_u32 {s(d)}, {s(d)}, {step}",
                f"s_addc_u32 {s(d + 1)}, {s(d + 1)}, 0",
                f"s_sub_i32 {s(d + 2)}, {s(d + 2)}, {step}",
                f"s_max_i32 {s(d + 2)}, {s(d + 2)}, 0"]
    return out


def rebase(base, delta):
    lit = hex(delta & 0xffffffff)
    return [ins(f"v_add_u32_e32 {v(base + i)}, {lit}, {v(base + i)}", "valu", dst=v(base + i), src=v(base + i))
            for i in range(8)]


def dp_part():
    """dS = P dP of the current block (P already in S), then the bf16 packs:
    h2 = 0 once phase-1 pair 7 has issued (MFMA 16), h2 = 1 after pair 15"""
    L = []
    order = [(kg, r) for r in range(16) for kg in range(2)]
    for kg, r in order:
        sv, dv = v(S + 16 * kg + r), v(DP + 16 * kg + r)
        L.append(ins(f"v_mul_f32_e32 {dv}, {sv}, {dv}", "valu", dst=dv, src=f"{sv} {dv}"))
    for h2 in range(2):
        for kg in range(2):
            for w in range(4):
                r = h2 * 8 + 2 * w
                for src, dst in ((S, PB), (DP, DSB)):
                    d = v(dst + kg * 8 + h2 * 4 + w)
                    x0, x1 = v(src + 16 * kg + r), v(src + 16 * kg + r + 1)
                    c = ins(f"v_cvt_pk_bf16_f32 {d}, {x0}, {x1}", "valu", dst=d, src=f"{x0} {x1}")
                    c.not_before = 16 if h2 == 0 else 32
                    L.append(c)
    return L


def s_part(gate):
    """P = exp2(S c) of the next block, clamped to [0, 1], after its S MFMAs"""
    L = []
    order = [(kg, r) for r in range(16) for kg in range(2)]
    mul = {e: ins(f"v_mul_f32_e32 {v(S + 16 * e[0] + e[1])}, %[c2], {v(S + 16 * e[0] + e[1])}", "valu",
                  dst=v(S + 16 * e[0] + e[1]), src=v(S + 16 * e[0] + e[1])) for e in order}
    ex = {e: ins(f"v_exp_f32_e64 {v(S + 16 * e[0] + e[1])}, {v(S + 16 * e[0] + e[1])} clamp", "trans",
                 dst=v(S + 16 * e[0] + e[1]), src=v(S + 16 * e[0] + e[1])) for e in order}
    n = len(order)
    for k in range(n + 2):  # exp two elements behind its multiply
        if k < n:
            L.append(mul[order[k]])
        if 0 <= k - 2 < n:
            L.append(ex[order[k - 2]])
    for i in L:
        i.not_before = gate
    return L


P2 = 32          # first phase-2 MFMA
DMA_AT = (1, 7, 13, 19, 25, 29)
SPLIT = 32       # the next block's first SPLIT exp-chain instructions run in this slot, the rest in the next


def r_base(u):
    """base buffer of RADDR in slot u, which reads block J + 1's rows (buffer u + 1)"""
    return 0 if (u + 1) % NBUF == 0 else 1


def t_base(u):
    """base buffer of TADDR in slot u's phase 1, which reads block J - 1's (buffer u - 1)"""
    return 0 if (u - 1) % NBUF < NBUF - 1 else 1


TADDR_BUF0 = t_base(0)  # where the kernel points TADDR (slot 0 reads buffer NBUF - 1: block -1, zeros)


def slot_body(u, entry):
    """slot J (J % 5 == u): RADDR reads block J + 1's buffer, TADDR block J - 1's"""
    rbuf, dmabuf = (u + 1) % NBUF, (u + AHEAD) % NBUF
    trel, rrel = (u - 1) % NBUF - t_base(u), rbuf - r_base(u)
    nt = (u + 1) % NBUF  # the next slot
    em = Emitter.merged_entry(entry)
    mf_list = []
    for n in range(16):
        mf_list += p1_pair(n)
    for m in range(16):
        mf_list += p2_pair(m)
    pinned = {}

    def pin(k, lst):
        pinned.setdefault(k, []).extend(lst)
    for n in range(2, 16):
        pin(2 * (n - 2), t_read(n, trel))
    pin(2, init_reads(rbuf))
    for i, at in enumerate(DMA_AT):
        pin(at, dma(i, dmabuf))
    pin(28, a_read(0, rrel))
    pin(30, a_read(1, rrel))
    for m in range(2, 16):
        pin(P2 + 2 * (m - 2), a_read(m, rrel))
    pin(P2 + 8, v_reads(0))
    pin(P2 + 12, v_reads(1))
    for ks in range(2, 8):
        pin(P2 + 2 * (8 + ks - 1), v_reads(ks))
    # TADDR to the next slot's base (when it changes), then the next slot's
    # first two fragments (block J, buffer u)
    if t_base(nt) != t_base(u):
        pin(P2, rebase(TADDR, (t_base(nt) - t_base(u)) * BUF))
    pin(P2 + 18, t_read(0, u - t_base(nt)))
    pin(P2 + 22, t_read(1, u - t_base(nt)))
    # RADDR to the next slot's base after the last row read
    if r_base(nt) != r_base(u):
        pin(P2 + 30, rebase(RADDR, (r_base(nt) - r_base(u)) * BUF))
    fillers = s_part(0)[SPLIT:] + dp_part() + s_part(P2 + 16)[:SPLIT]
    left = fill_schedule(em, mf_list, fillers, budget=BUDGET, pinned=pinned, flush_war=True)
    em.emit_all(left)
    return em


def prologue():
    em = Emitter()
    for r in range(PB, DSB + 16):  # P, dS of block -1: zero
        em.raw(f"v_mov_b32 {v(r)}, 0", 1)
    for r in range(256):
        em.raw(f"v_accvgpr_write_b32 {a(r)}, 0", 1)
    em.raw("s_cmp_eq_u32 %[nb], 0")
    em.raw(f"s_cbranch_scc1 {lbl('done')}")
    for d, p, nr in ((DQ, "%[qp]", "%[qnr]"), (DG, "%[gp]", "%[gnr]"), (DS0, "%[sp0]", "%[snr]"),
                     (DS1, "%[sp1]", "%[snr]")):
        for line in (f"s_mov_b64 {s(d, 2)}, {p}", f"s_mov_b32 {s(d + 2)}, {nr}", f"s_mov_b32 {s(d + 3)}, 0x20000"):
            em.raw(line, 1)
    em.raw(f"s_mov_b32 {s(J)}, 0", 1)
    for blk in range(AHEAD):
        for i in range(6):
            em.emit_all(dma(i, blk))
        for line in desc_advance():
            em.raw(line, 1)
    em.raw(f"s_waitcnt vmcnt({6 * (AHEAD - 1)})")  # block 0 (this wave's part)
    em.raw("s_barrier")
    em.emit_all(init_reads(0))
    mfl = []
    for m in range(16):
        mfl += p2_pair(m)
    pinned = {0: a_read(0, 0) + a_read(1, 0) + v_reads(0) + v_reads(1)}
    for m in range(2, 16):
        pinned.setdefault(2 * (m - 2), []).extend(a_read(m, 0))
    for ks in range(2, 8):
        pinned.setdefault(2 * (8 + ks - 1), []).extend(v_reads(ks))
    left = fill_schedule(em, mfl, s_part(16)[:SPLIT], budget=BUDGET, pinned=pinned)
    em.emit_all(left)
    # slot 0 reads S / dP rows from buffer 1 (RADDR to its base); its dV / dK
    # fragments (block -1, zeros) from buffer NBUF - 1
    em.emit_all(rebase(RADDR, r_base(0) * BUF))
    em.emit_all(t_read(0, NBUF - 1 - TADDR_BUF0) + t_read(1, NBUF - 1 - TADDR_BUF0))
    return em


def final_dvdk(u, entry):
    """dV / dK of the last block after its slot u: P / dS packed there, TADDR
    at the next slot's base, the first two fragments read"""
    em = Emitter.merged_entry(entry)
    mfl = []
    for n in range(16):
        mfl += p1_pair(n)
    pinned = {}
    for n in range(2, 16):
        pinned.setdefault(2 * (n - 2), []).extend(t_read(n, u - t_base((u + 1) % NBUF)))
    fill_schedule(em, mfl, [], pinned=pinned)
    em.settle()
    return em


def build():
    """The loop's lines."""
    pro = prologue()
    bodies, ends = {}, {u: [] for u in range(NBUF)}
    for _ in range(4):
        new = {}
        for u in range(NBUF):
            prev = ends[(u - 1) % NBUF] + ([pro] if u == 0 else [])
            new[u] = slot_body(u, prev or [pro])
        bodies = new
        ends = {u: [bodies[u]] for u in range(NBUF)}
    lines = list(pro.lines)
    lines.append(f"{lbl('loop')}:")
    for u in range(NBUF):
        # issued: blocks up to J + 2; block J + 1 (this slot's S / dP rows and
        # statistics) must have landed for every wave
        lines += [f"s_waitcnt vmcnt({6 * (AHEAD - 2)})", "s_barrier"]
        lines += bodies[u].lines
        lines += desc_advance()
        lines.append(f"s_add_u32 {s(J)}, {s(J)}, 1")
        lines.append(f"s_cmp_eq_u32 {s(J)}, %[nb]")
        lines.append(f"s_cbranch_scc1 {lbl(f'exit{u}')}")
    lines.append(f"s_branch {lbl('loop')}")
    for u in range(NBUF):
        lines.append(f"{lbl(f'exit{u}')}:")
        lines += final_dvdk(u, [bodies[u]]).lines
        lines.append(f"s_branch {lbl('done')}")
    lines.append(f"{lbl('done')}:")
    lines.append("s_waitcnt vmcnt(0) lgkmcnt(0)")
    return lines


def render(lines):
    def body(ls):
        return " \\\n".join('  "' + ln + '\\n\\t"' for ln in ls)
    return ("// Generated by dkdv_asm_gen.py: the main loop of dkdv_asm_kernel (dkdv_asm.hip).\n"
            "// Do not edit; change the generator and rebuild.\n"
            "#pragma once\n"
            f"#define HARP_DKDV_ASM_SGPR_CLOBBERS {clobber_list(SGPR_CLOBBER)}\n"
            f"#define HARP_DKDV_ASM_LOOP \\\n{body(lines)}\n")


def write(path=None):
    path = path or os.path.join(os.path.dirname(os.path.abspath(__file__)), "dkdv_asm.inc")
    text = render(build())
    old = open(path).read() if os.path.exists(path) else None
    if old != text:
        with open(path, "w") as f:
            f.write(text)
    return path


if __name__ == "__main__":
    p = write()
    print(p, sum(1 for _ in open(p)), "lines")
