"""Generator of the hand-scheduled main loop of fwd_asm_kernel (fwd_asm.hip),
written to fwd_asm.inc as one inline-asm string (HARP_FWD_ASM_LOOP).

Run by harp_amd/build.py before compiling; `python fwd_asm_gen.py` rewrites
the file by hand.

Work split: a block of 4 waves x 64 queries (one wave per SIMD), D = 128.  A
wave's queries form two 32-query groups qg; every K / V fragment read from LDS
feeds one MFMA per group (0.5 KB of LDS per MFMA).  Keys are streamed in
32-key blocks J through eight 16 KiB LDS block buffers (K at 8 KiB * (J % 8),
V at 64 KiB + 8 KiB * (J % 8)), copied global -> LDS by buffer_load ... lds
five blocks ahead of their use.  A barrier before every even slot J publishes
blocks J + 1 and J + 2 and shows that every wave is done with slot J - 1, so
the copies of slots J and J + 1 may go into the buffers of blocks J - 3 and
J - 2.

Slot J (one per key block):
  MFMAs  O(J-1) += V(J-1)^T P^T(J-1)   (a0..a127, 16 MFMAs)
         S(J+1)  = K(J+1) Q^T          (16 MFMAs, Q in a128..a191)
  VALU   online softmax of S(J): P(J) = bf16 of exp2(S c2 - m_ref) against
         the lane's current reference point m_ref, row sums (fp32, unrounded
         exps), and the rescale check: a lane whose 16 exps of the block sum
         above 2^8 (some key above m_ref + 8 in log2 units, or the first keys
         of a row, whose m_ref is still -FLT_MAX and whose exps overflow)
         flags the wave
  copies of block J + 5 (4 per wave)
The loop is unrolled over the eight buffers; each slot has a masked twin
(keys past a chunk's valid length set to -inf) entered when its block is a
chunk's partial last one, and an out-of-line rescale (one per slot parity):
m_ref moves up to the row's maximum over block J (both lane halves), O and l
are multiplied by 2^(old - new), and P(J) and the block sums are computed
again from S(J), which the exps leave intact.  The kernel writes m_ref as the
row statistic m, with l relative to it: m + log l is the row's LSE (what the
backward reads); m is within 8 log2 units below the row's exact maximum.
The reference math is ring_attn.cpp:2412-2575 (ring_attention_forward).
"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from asm_sched import Emitter, clobber_list, fill_schedule, ins, regs_of  # noqa: E402

# ---- registers ------------------------------------------------------------
KADDR, VADDR, DOFF = 32, 40, 48          # per-lane LDS addresses / copy offsets
MREF, MMAX, LRUN, LSUM, MNEW, MX = 50, 52, 54, 56, 58, 60  # pairs (qg); MMAX unused
KF, VF = 64, 80                          # 4 fragment buffers x 4 registers each
P = (96, 112)                            # P[par]: qg * 8 + k2 * 4 + w
S = (128, 160)                           # S[par]: qg * 16 + r
LIM, G4, NEGV, TMP, CORR = 192, 193, 194, 196, 204  # misc2 tuple v192..v223
ET, NET = 206, 12                        # ring of exp temporaries v206..v217 (misc2)
AQ = 128                                 # Q in a128..a191: (qg * 8 + ks) * 4
# SGPRs (clobbered by the asm statement)
F, FLAG, MK = (60, 62), 64, (66, 68)
DK, DV = 72, 76
# the copy cursor: the K / V row pointers of the next block are words 0-1 of DK / DV
LEFT, STEP, CH, T0, T1, VAL, VALJ, RING, J, U = 84, 85, 86, 87, 88, 90, 91, (92, 93), 94, 95
SGPR_CLOBBER = list(range(60, 96))

NEG_BIG = "0xff7fffff"  # -FLT_MAX
SKEW_EXP, SKEW_ADD = 4, 8  # softmax pipeline: element k's exp and sum trail its FMA by this many elements
LIMIT = "0x43800000"    # 256.0 = 2^8: a lane's block sum above it triggers the rescale


def v(r, n=1):
    return f"v{r}" if n == 1 else f"v[{r}:{r + n - 1}]"


def a(r, n=1):
    return f"a{r}" if n == 1 else f"a[{r}:{r + n - 1}]"


def s(r, n=1):
    return f"s{r}" if n == 1 else f"s[{r}:{r + n - 1}]"


def lbl(name):
    return f".Lfa_{name}_%="


# ---- pieces of a slot -----------------------------------------------------
def mfma_o(i, par):
    """O pair i (db = i // 2, k2 = i % 2), V^T fragment in VF[i % 4]"""
    db, k2 = i // 2, i % 2
    po = P[1 - par]
    out = []
    for qg in range(2):
        acc = a(64 * qg + 16 * db, 16)
        b = v(po + qg * 8 + k2 * 4, 4)
        frag = v(VF + 4 * (i % 4), 4)
        out.append(ins(f"v_mfma_f32_32x32x16_bf16 {acc}, {frag}, {b}, {acc}", "mfma", dst=acc, src=f"{frag} {b}",
                       srcC=acc))
    return out


def mfma_s(ks, par):
    nxt = S[1 - par]
    out = []
    for qg in range(2):
        acc = v(nxt + 16 * qg, 16)
        b = a(AQ + (qg * 8 + ks) * 4, 4)
        frag = v(KF + 4 * (ks % 4), 4)
        c = "0" if ks == 0 else acc
        out.append(ins(f"v_mfma_f32_32x32x16_bf16 {acc}, {frag}, {b}, {c}", "mfma", dst=acc, src=f"{frag} {b}",
                       srcC=(acc if ks else "")))
    return out


def ds_k(ks, kbuf):
    frag = v(KF + 4 * (ks % 4), 4)
    return [ins(f"ds_read_b128 {frag}, {v(KADDR + ks)} offset:{kbuf * 8192}", "ds", dst=frag, src=v(KADDR + ks))]


def ds_v(i, vbuf):
    db, k2 = i // 2, i % 2
    f = VF + 4 * (i % 4)
    off = vbuf * 8192 + k2 * 4096
    return [ins(f"ds_read_b64_tr_b16 {v(f, 2)}, {v(VADDR + db)} offset:{off}", "ds", dst=v(f, 2), src=v(VADDR + db)),
            ins(f"ds_read_b64_tr_b16 {v(f + 2, 2)}, {v(VADDR + 4 + db)} offset:{off}", "ds", dst=v(f + 2, 2),
                src=v(VADDR + 4 + db))]


def dma(i, dmabuf):
    """copy instruction i of a block (0, 1: K rows; 2, 3: V rows) into buffer dmabuf"""
    kv = i // 2
    base = (0 if kv == 0 else 65536) + dmabuf * 8192 + (i % 2) * 1024
    desc = s(DK, 4) if kv == 0 else s(DV, 4)
    return [ins(f"s_add_u32 m0, %[dbase], {base}", "m0", dst=["m0"]),
            ins(f"buffer_load_dwordx4 {v(DOFF + i % 2)}, {desc}, 0 offen lds", "vmem", src=[v(DOFF + i % 2), "m0"])]


def exp_pipeline(par):
    """P(par) = bf16 of exp2(S(par) c2 - m_ref) and the block sums LSUM, the
    exps in the temporaries ET.. (S stays intact), skewed: fma(k),
    exp(k - SKEW_EXP), add / pack(k - SKEW_ADD).  Element k's temporary is
    last read by the pack of element k + 2, before element k + NET's fma."""
    cur, pn = S[par], P[par]
    sv = lambda qg, r: v(cur + 16 * qg + r)
    order = [(qg, r) for r in range(16) for qg in range(2)]
    tv = {e: v(ET + k % NET) for k, e in enumerate(order)}
    fmas = {e: ins(f"v_fma_f32 {tv[e]}, {sv(*e)}, %[c2], -{v(MREF + e[0])}", "valu", dst=tv[e],
                   src=f"{sv(*e)} {v(MREF + e[0])}") for e in order}
    exps = {e: ins(f"v_exp_f32_e32 {tv[e]}, {tv[e]}", "trans", dst=tv[e], src=tv[e]) for e in order}
    adds, cvts = {}, {}
    for (qg, r) in order:
        if r == 1:
            adds[(qg, r)] = ins(f"v_add_f32_e32 {v(LSUM + qg)}, {tv[(qg, 0)]}, {tv[(qg, 1)]}", "valu",
                                dst=v(LSUM + qg), src=f"{tv[(qg, 0)]} {tv[(qg, 1)]}")
        elif r > 1:
            adds[(qg, r)] = ins(f"v_add_f32_e32 {v(LSUM + qg)}, {v(LSUM + qg)}, {tv[(qg, r)]}", "valu",
                                dst=v(LSUM + qg), src=f"{v(LSUM + qg)} {tv[(qg, r)]}")
        if r % 2 == 1:
            k2, j = r // 8, (r - 1) % 8
            dst = v(pn + qg * 8 + k2 * 4 + j // 2)
            cvts[(qg, r)] = ins(f"v_cvt_pk_bf16_f32 {dst}, {tv[(qg, r - 1)]}, {tv[(qg, r)]}", "valu", dst=dst,
                                src=f"{tv[(qg, r - 1)]} {tv[(qg, r)]}")
    L = []
    n = len(order)
    for k in range(n + SKEW_ADD + 2):
        if k < n:
            L.append(fmas[order[k]])
        if 0 <= k - SKEW_EXP < n:
            L.append(exps[order[k - SKEW_EXP]])
        if 0 <= k - SKEW_ADD < n:
            e = order[k - SKEW_ADD]
            if e in adds:
                L.append(adds[e])
            if e in cvts:
                L.append(cvts[e])
    return L


def softmax(par, masked):
    cur = S[par]
    L = []
    sv = lambda qg, r: v(cur + 16 * qg + r)
    for qg in range(2):  # the previous block's row sums (relative to the current reference)
        L.append(ins(f"v_add_f32_e32 {v(LRUN + qg)}, {v(LRUN + qg)}, {v(LSUM + qg)}", "valu", dst=v(LRUN + qg),
                     src=f"{v(LRUN + qg)} {v(LSUM + qg)}"))
    if masked:  # keys c_row(r, g) = 8 (r / 4) + 4 g + r % 4 >= valid  ->  -inf;  LIM = valid - 4 g
        for r in range(16):
            k = 8 * (r // 4) + r % 4
            L.append(ins(f"v_cmp_ge_i32_e32 vcc, {k}, {v(LIM)}", "valu", dst=["vcc"], src=v(LIM)))
            for qg in range(2):
                L.append(ins(f"v_cndmask_b32_e32 {sv(qg, r)}, {sv(qg, r)}, {v(NEGV)}, vcc", "valu", dst=sv(qg, r),
                             src=[*[sv(qg, r)], v(NEGV), "vcc"]))
    L += exp_pipeline(par)
    for qg in range(2):  # a block sum above 2^8 (or inf) flags the wave for the rescale; NaN does not
        L.append(ins(f"v_cmp_lt_f32_e32 vcc, {LIMIT}, {v(LSUM + qg)}", "valu", dst=["vcc"], src=v(LSUM + qg)))
        L.append(ins(f"s_or_b64 {s(FLAG, 2)}, {s(FLAG, 2)}, vcc", "salu", dst=s(FLAG, 2),
                     src=[*regs_of(s(FLAG, 2)), "vcc"]))
    return L


PAIR_ORDER = ["O0", "O1", "S0", "O2", "S1", "O3", "S2", "O4", "S3", "O5", "S4", "O6", "S5", "S6", "S7", "O7"]
DMA_AT = (1, 9, 17, 25)
BUDGET = 20


def slot_body(u, entry, masked):
    """The scheduled body of slot J (J % 8 == u): returns its Emitter."""
    par, kbuf, vbuf, vnext, dmabuf = u % 2, (u + 1) % 8, (u + 7) % 8, u, (u + 5) % 8
    em = Emitter.merged_entry(entry)
    mf, idx, pinned = [], {}, {}
    for p in PAIR_ORDER:
        idx[p] = len(mf)
        mf += mfma_o(int(p[1]), par) if p[0] == "O" else mfma_s(int(p[1]), par)
    pre = []
    for ks in range(4):
        pre += ds_k(ks, kbuf)
    pinned[0] = pre + ds_v(2, vbuf) + ds_v(3, vbuf)
    for ks in range(4, 8):
        pinned.setdefault(idx[f"S{ks - 4}"] + 2, []).extend(ds_k(ks, kbuf))
    for i in range(4, 8):
        pinned.setdefault(idx[f"O{i - 4}"] + 2, []).extend(ds_v(i, vbuf))
    pinned.setdefault(idx["O4"] + 2, []).extend(ds_v(0, vnext))  # the next slot's first two V fragments
    pinned.setdefault(idx["O5"] + 2, []).extend(ds_v(1, vnext))
    for i, at in enumerate(DMA_AT):
        pinned.setdefault(at, []).extend(dma(i, dmabuf))
    left = fill_schedule(em, mf, softmax(par, masked), budget=BUDGET, pinned=pinned)
    em.emit_all(left)
    return em


def cursor_desc(block_ring_slot):
    """Descriptors of the block at the cursor (DK / DV words 2 = its bytes
    left in the chunk) and its valid key count into the ring."""
    w = block_ring_slot
    sh, rg = (w % 4) * 8, RING[w // 4]
    return [
        f"s_max_i32 {s(T0)}, {s(LEFT)}, 0",
        f"s_min_u32 {s(VAL)}, {s(T0)}, 32",
        f"s_mul_i32 {s(DK + 2)}, {s(T0)}, %[sbytes]",
        f"s_mov_b32 {s(DV + 2)}, {s(DK + 2)}",
        f"s_lshl_b32 {s(T1)}, {s(VAL)}, {sh}",
        f"s_and_b32 {s(rg)}, {s(rg)}, {hex(0xffffffff ^ (0xff << sh))}",
        f"s_or_b32 {s(rg)}, {s(rg)}, {s(T1)}",
    ]


def cursor_adv(tag):
    """Move the cursor 32 keys on (after the block's copies are issued): into
    the next non-empty chunk of the split when this one ends.  Row pointers
    stay below 2^48, so words 1 of DK / DV keep a zero stride field."""
    return [
        f"s_add_u32 {s(DK)}, {s(DK)}, %[blkb]",
        f"s_addc_u32 {s(DK + 1)}, {s(DK + 1)}, 0",
        f"s_add_u32 {s(DV)}, {s(DV)}, %[blkb]",
        f"s_addc_u32 {s(DV + 1)}, {s(DV + 1)}, 0",
        f"s_sub_i32 {s(LEFT)}, {s(LEFT)}, 32",
        f"s_cmp_gt_i32 {s(LEFT)}, 0",
        f"s_cbranch_scc1 {lbl('cok' + tag)}",
        f"{lbl('cadv' + tag)}:",
        f"s_add_i32 {s(STEP)}, {s(STEP)}, 1",
        f"s_cmp_ge_i32 {s(STEP)}, %[end]",
        f"s_cbranch_scc1 {lbl('cexh' + tag)}",
        f"s_lshl_b32 {s(T0)}, {s(STEP)}, 2",
        f"s_add_u32 {s(T0)}, {s(T0)}, %[ooff]",
        f"s_load_dword {s(CH)}, %[ctp], {s(T0)}",
        "s_waitcnt lgkmcnt(0)",
        f"s_lshl_b32 {s(T0)}, {s(CH)}, 2",
        f"s_add_u32 {s(T0)}, {s(T0)}, %[loff]",
        f"s_load_dword {s(LEFT)}, %[ctp], {s(T0)}",
        f"s_lshl_b32 {s(T1)}, {s(CH)}, 3",
        f"s_add_u32 {s(T0)}, {s(T1)}, %[koff]",
        f"s_load_dwordx2 {s(DK, 2)}, %[ctp], {s(T0)}",
        f"s_add_u32 {s(T0)}, {s(T1)}, %[voff]",
        f"s_load_dwordx2 {s(DV, 2)}, %[ctp], {s(T0)}",
        "s_waitcnt lgkmcnt(0)",
        f"s_cmp_le_i32 {s(LEFT)}, 0",
        f"s_cbranch_scc1 {lbl('cadv' + tag)}",
        f"s_add_u32 {s(DK)}, {s(DK)}, %[kvl]",
        f"s_addc_u32 {s(DK + 1)}, {s(DK + 1)}, %[kvh]",
        f"s_add_u32 {s(DV)}, {s(DV)}, %[kvl]",
        f"s_addc_u32 {s(DV + 1)}, {s(DV + 1)}, %[kvh]",
        f"s_branch {lbl('cok' + tag)}",
        f"{lbl('cexh' + tag)}:",
        f"s_mov_b32 {s(LEFT)}, 0",
        f"{lbl('cok' + tag)}:",
    ]


def prologue():
    em = Emitter()
    # fragments, P (P(-1) = 0) and O start at zero; a split without keys ends here
    for r in range(KF, P[1] + 16):
        em.raw(f"v_mov_b32 {v(r)}, 0", 1)
    for r in range(128):
        em.raw(f"v_accvgpr_write_b32 {a(r)}, 0", 1)
    for qg in range(2):  # m_ref: the first keys of a row overflow their exps and so flag the rescale
        em.raw(f"v_mov_b32 {v(MREF + qg)}, {NEG_BIG}", 1)
    em.raw("s_cmp_eq_u32 %[nb], 0")
    em.raw(f"s_cbranch_scc1 {lbl('done')}")
    em.raw("s_waitcnt lgkmcnt(0)")  # the zero fill of V buffer 7 (O(-1) reads it with P = 0)
    for line in (f"s_mov_b32 {s(DK + 3)}, 0x20000", f"s_mov_b32 {s(DV + 3)}, 0x20000",
                 f"s_mov_b64 {s(DK, 2)}, %[kp0]", f"s_mov_b64 {s(DV, 2)}, %[vp0]", f"s_mov_b32 {s(LEFT)}, %[left0]",
                 f"s_mov_b32 {s(STEP)}, %[step0]", f"s_mov_b32 {s(RING[0])}, 0", f"s_mov_b32 {s(RING[1])}, 0",
                 f"s_mov_b32 {s(J)}, 0", f"s_mov_b64 {s(FLAG, 2)}, 0"):
        em.raw(line, 1)
    for b in range(5):
        for line in cursor_desc(b):
            em.raw(line, 1)
        for i in range(4):
            em.emit_all(dma(i, b))
        for line in cursor_adv(f"p{b}"):
            em.raw(line, 1)
    em.raw("s_waitcnt vmcnt(16)")  # block 0 (this wave's part)
    em.raw("s_barrier")
    mf = []
    for ks in range(8):
        mf += mfma_s(ks, 1)  # writes S[0]: slot 0 (par 0) reads it as its current block
    pinned = {0: ds_k(0, 0) + ds_k(1, 0) + ds_k(2, 0) + ds_k(3, 0)}
    for ks in range(4, 8):
        pinned[2 * (ks - 4) + 2] = ds_k(ks, 0)
    pinned[12] = ds_v(0, 7) + ds_v(1, 7)  # slot 0's O(-1) fragments (zeros, P(-1) = 0)
    fill_schedule(em, mf, [], pinned=pinned)
    return em


def rescale(par):
    """After slot J (parity par) flagged: m_ref moves to the larger of itself
    and c2 times the row's maximum over block J (both lane halves), O and l
    are multiplied by corr = 2^(m_ref - m_new) (m_new >= m_ref: 1 where
    unchanged, 0 from -FLT_MAX), and P(J) and the block sums are computed
    again against the new reference from S(J).  Blocks that did not flag
    have every exp at most 2^8 (their sums are), so every score seen so far
    stays within 8 (log2 units) above the new m_ref."""
    em = Emitter()
    em.nop(16)  # the last O MFMAs of the slot
    m0, m1 = v(MX), v(MX + 1)
    cur = S[par]
    for qg in range(2):  # the lane's maximum of block J's raw scores (masked keys are -inf)
        sv = lambda r: v(cur + 16 * qg + r)
        mx = v(MX + qg)
        em.emit(ins(f"v_max_f32_e32 {mx}, {sv(0)}, {sv(1)}", "valu", dst=mx, src=f"{sv(0)} {sv(1)}"))
        for r in range(2, 16, 2):
            em.emit(ins(f"v_max3_f32 {mx}, {mx}, {sv(r)}, {sv(r + 1)}", "valu", dst=mx,
                        src=f"{mx} {sv(r)} {sv(r + 1)}"))
    # [mx0 lo | mx0 hi], [mx1 lo | mx1 hi] -> swap, max -> [M0 | M1] -> copy, swap -> [M0 | M0], [M1 | M1]
    em.emit(ins(f"v_permlane32_swap_b32_e32 {m0}, {m1}", "perm", dst=f"{m0} {m1}", src=f"{m0} {m1}"))
    em.emit(ins(f"v_max_f32_e32 {m0}, {m0}, {m1}", "valu", dst=m0, src=f"{m0} {m1}"))
    em.emit(ins(f"v_mov_b32_e32 {m1}, {m0}", "valu", dst=m1, src=m0))
    em.emit(ins(f"v_permlane32_swap_b32_e32 {m0}, {m1}", "perm", dst=f"{m0} {m1}", src=f"{m0} {m1}"))
    for qg in range(2):
        mn, t, c = v(MNEW + qg), v(TMP + qg), v(CORR + qg)
        em.emit(ins(f"v_mul_f32_e32 {mn}, %[c2], {v(MX + qg)}", "valu", dst=mn, src=v(MX + qg)))
        em.emit(ins(f"v_max_f32_e32 {mn}, {v(MREF + qg)}, {mn}", "valu", dst=mn, src=f"{v(MREF + qg)} {mn}"))
        em.emit(ins(f"v_sub_f32_e32 {t}, {v(MREF + qg)}, {mn}", "valu", dst=t, src=f"{v(MREF + qg)} {mn}"))
        em.emit(ins(f"v_exp_f32_e32 {c}, {t}", "trans", dst=c, src=t))
    for qg in range(2):
        c = v(CORR + qg)
        em.emit(ins(f"v_mul_f32_e32 {v(LRUN + qg)}, {v(LRUN + qg)}, {c}", "valu", dst=v(LRUN + qg),
                    src=f"{v(LRUN + qg)} {c}"))
        em.emit(ins(f"v_mov_b32_e32 {v(MREF + qg)}, {v(MNEW + qg)}", "valu", dst=v(MREF + qg), src=v(MNEW + qg)))
    for base in range(0, 128, 8):
        qg = base // 64
        for k in range(8):
            t = v(TMP + k)
            em.emit(ins(f"v_accvgpr_read_b32 {t}, {a(base + k)}", "valu", dst=t, src=a(base + k)))
        for k in range(8):
            t = v(TMP + k)
            em.emit(ins(f"v_mul_f32_e32 {t}, {t}, {v(CORR + qg)}", "valu", dst=t, src=f"{t} {v(CORR + qg)}"))
        for k in range(8):
            t = v(TMP + k)
            em.emit(ins(f"v_accvgpr_write_b32 {a(base + k)}, {t}", "valu", dst=a(base + k), src=t))
    em.emit_all(exp_pipeline(par))
    em.nop(4)
    return em


def final_o(u, entry):
    """O(NB-1) after the last slot (J - 1 = NB - 1, J % 8 == u + 1): P[u % 2],
    V buffer u; its first two fragments were prefetched by slot u."""
    par_next = (u + 1) % 2  # the O MFMAs read P[1 - par] of a slot with par = (u + 1) % 2
    em = Emitter.merged_entry(entry)
    mf = []
    pinned = {0: ds_v(2, u) + ds_v(3, u)}
    for i in range(8):
        mf += mfma_o(i, par_next)
    for i in range(4, 8):
        pinned[2 * (i - 4) + 2] = ds_v(i, u)
    fill_schedule(em, mf, [], pinned=pinned)
    for qg in range(2):
        em.emit(ins(f"v_add_f32_e32 {v(LRUN + qg)}, {v(LRUN + qg)}, {v(LSUM + qg)}", "valu", dst=v(LRUN + qg),
                    src=f"{v(LRUN + qg)} {v(LSUM + qg)}"))
    em.settle()
    return em


def build():
    """The loop's lines."""
    pro = prologue()
    resc = (rescale(0), rescale(1))
    # fixed point of the slot boundary states: slot u is entered from slot
    # u - 1 (plain, masked or through the rescale), slot 0 also from the
    # prologue
    bodies = {}
    ends = {u: [] for u in range(8)}
    for _ in range(4):
        new = {}
        for u in range(8):
            prev = ends[(u - 1) % 8] + ([pro] if u == 0 else [])
            new[u] = (slot_body(u, prev or [pro], False), slot_body(u, prev or [pro], True))
        bodies = new
        ends = {u: [bodies[u][0], bodies[u][1], resc[u % 2]] for u in range(8)}
    lines = []
    lines += pro.lines
    lines.append(f"{lbl('loop')}:")
    for u in range(8):
        if u % 2 == 0:
            lines += ["s_waitcnt vmcnt(8)", "s_barrier"]
        lines += cursor_desc((u + 5) % 8)
        lines.append(f"s_bfe_u32 {s(VALJ)}, {s(RING[u // 4])}, {hex(((u % 4) * 8) | (8 << 16))}")
        lines.append(f"s_cmp_lt_u32 {s(VALJ)}, 32")
        lines.append(f"s_cbranch_scc1 {lbl(f'mask{u}')}")
        lines += bodies[u][0].lines
        lines.append(f"{lbl(f'join{u}')}:")
        lines += cursor_adv(f"s{u}")
        lines.append(f"s_cmp_lg_u64 {s(FLAG, 2)}, 0")
        lines.append(f"s_cbranch_scc1 {lbl(f'resc{u}')}")
        lines.append(f"{lbl(f'ret{u}')}:")
        lines.append(f"s_add_u32 {s(J)}, {s(J)}, 1")
        lines.append(f"s_cmp_eq_u32 {s(J)}, %[nb]")
        lines.append(f"s_cbranch_scc1 {lbl(f'exit{u}')}")
    lines.append(f"s_branch {lbl('loop')}")
    for u in range(8):  # masked twins
        lines.append(f"{lbl(f'mask{u}')}:")
        lines.append(f"v_sub_u32_e32 {v(LIM)}, {s(VALJ)}, {v(G4)}")
        lines += bodies[u][1].lines
        lines.append(f"s_branch {lbl(f'join{u}')}")
    for u in range(8):
        lines.append(f"{lbl(f'resc{u}')}:")
        lines.append(f"s_mov_b32 {s(U)}, {u}")
        lines.append(f"s_branch {lbl(f'rescale{u % 2}')}")
    for par in range(2):
        lines.append(f"{lbl(f'rescale{par}')}:")
        lines += resc[par].lines
        lines.append(f"s_mov_b64 {s(FLAG, 2)}, 0")
        for u in range(par, 8, 2):
            lines.append(f"s_cmp_eq_u32 {s(U)}, {u}")
            lines.append(f"s_cbranch_scc1 {lbl(f'ret{u}')}")
    for u in range(8):
        lines.append(f"{lbl(f'exit{u}')}:")
        lines += final_o(u, [bodies[u][0], bodies[u][1], *resc]).lines
        lines.append(f"s_branch {lbl('done')}")
    lines.append(f"{lbl('done')}:")
    lines.append("s_waitcnt vmcnt(0) lgkmcnt(0)")
    return lines


def render(lines):
    def body(ls):
        return " \\\n".join('  "' + ln + '\\n\\t"' for ln in ls)
    return ("// Generated by fwd_asm_gen.py: the main loop of fwd_asm_kernel (fwd_asm.hip).\n"
            "// Do not edit; change the generator and rebuild.\n"
            "#pragma once\n"
            f"#define HARP_FWD_ASM_SGPR_CLOBBERS {clobber_list(SGPR_CLOBBER)}\n"
            f"#define HARP_FWD_ASM_LOOP \\\n{body(lines)}\n")


def write(path=None):
    path = path or os.path.join(os.path.dirname(os.path.abspath(__file__)), "fwd_asm.inc")
    text = render(build())
    old = open(path).read() if os.path.exists(path) else None
    if old != text:
        with open(path, "w") as f:
            f.write(text)
    return path


if __name__ == "__main__":
    p = write()
    print(p, sum(1 for _ in open(p)), "lines")
