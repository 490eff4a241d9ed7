"""Generator of the hand-scheduled main loop of dq_asm_kernel (dq_asm.hip),
written to dq_asm.inc as one inline-asm string (HARP_DQ_ASM_LOOP).

Run by harp_amd/build.py before compiling; `python dq_asm_gen.py` rewrites
the file by hand.

Work split as in the forward's loop (fwd_asm_gen.py): a block of 4 waves x 64
queries (one wave per SIMD), D = 128, two 32-query groups per wave, so every
K, V or K^T fragment read from LDS feeds two MFMAs.  AGPRs hold dQ^T
(a0..a127), Q (a128..a191) and dO (a192..a255), the B operands of S^T and
dP^T.  Keys stream in 32-key blocks through the same eight LDS block buffers,
copied five blocks ahead, with a barrier before every even slot.

Slot J:
  MFMAs  dQ^T(J-1) += K^T(J-1) dS^T(J-1)  (16)
         S^T(J+1) = K(J+1) Q^T, dP^T(J+1) = V(J+1) dO^T - D  (16 + 16; the
         dP^T accumulators start from -D of the lane's query, in v0..v31)
  VALU   P = exp2(S^T c2 - LSE2) clamped to [0, 1], dS^T = P (dP^T - D) of
         block J, rounded to bf16 after the dQ MFMAs have read the previous
         block's dS^T
  copies of block J + 5
Pad keys (past a chunk's valid length) load as zero K / V rows: their dS^T
meets a zero K^T row, so no mask is needed; the clamp keeps their P finite.
The reference math is ring_attn.cpp:2577-2829 (ring_attention_backward: dQ
from dS and K), as dq_kernel in ra_kernels.hip computes it.
"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from asm_sched import Emitter, clobber_list, fill_schedule, ins  # noqa: E402
from fwd_asm_gen import (DK, DV, FLAG, J, LEFT, RING, SGPR_CLOBBER, STEP, a, cursor_adv, cursor_desc,  # noqa: E402
                         lbl, s, v)

# ---- registers ------------------------------------------------------------
KADDR, VADDR, TADDR, DOFF = 32, 40, 48, 56   # per-lane LDS addresses / copy offsets
LSE = 58                                     # pair (qg): LSE2 of the lane's query
NEGD = 0                                     # v0..v31: -D of the lane's query, 16 copies per qg (the
                                             # initial dP^T accumulator, so dP - D needs no VALU)
KF, VF, TF = 64, 80, 96                      # 4 fragment buffers x 4 registers each
DS = 112                                     # dS^T bf16: qg * 8 + k2 * 4 + w
S = (128, 160)                               # S^T[par]: qg * 16 + r
DP = (192, 224)                              # dP^T[par]
AQ, ADO = 128, 192


def mf_s(ks, par):
    out = []
    for qg in range(2):
        acc = v(S[1 - par] + 16 * qg, 16)
        fr, b = v(KF + 4 * (ks % 4), 4), a(AQ + (qg * 8 + ks) * 4, 4)
        out.append(ins(f"v_mfma_f32_32x32x16_bf16 {acc}, {fr}, {b}, {'0' if ks == 0 else acc}", "mfma", dst=acc,
                       src=f"{fr} {b}", srcC=(acc if ks else "")))
    return out


def mf_dp(ks, par):
    out = []
    for qg in range(2):
        acc = v(DP[1 - par] + 16 * qg, 16)
        fr, b = v(VF + 4 * (ks % 4), 4), a(ADO + (qg * 8 + ks) * 4, 4)
        c = v(NEGD + 16 * qg, 16) if ks == 0 else acc
        out.append(ins(f"v_mfma_f32_32x32x16_bf16 {acc}, {fr}, {b}, {c}", "mfma", dst=acc, src=f"{fr} {b}",
                       srcC=c))
    return out


def mf_dq(i):
    """dQ pair i (db = i // 2, k2 = i % 2): K^T fragment in TF[i % 4]"""
    db, k2 = i // 2, i % 2
    out = []
    for qg in range(2):
        acc = a(64 * qg + 16 * db, 16)
        fr, b = v(TF + 4 * (i % 4), 4), v(DS + qg * 8 + k2 * 4, 4)
        out.append(ins(f"v_mfma_f32_32x32x16_bf16 {acc}, {fr}, {b}, {acc}", "mfma", dst=acc, src=f"{fr} {b}",
                       srcC=acc))
    return out


def ds_row(base, buf_reg, ks, off):
    fr = v(buf_reg + 4 * (ks % 4), 4)
    return [ins(f"ds_read_b128 {fr}, {v(base + ks)} offset:{off}", "ds", dst=fr, src=v(base + ks))]


def ds_t(i, buf):
    """K^T fragment of dQ pair i: rows 16 k2 .. of block buffer buf, d block db"""
    db, k2 = i // 2, i % 2
    f = TF + 4 * (i % 4)
    off = buf * 8192 + k2 * 4096
    return [ins(f"ds_read_b64_tr_b16 {v(f, 2)}, {v(TADDR + db)} offset:{off}", "ds", dst=v(f, 2), src=v(TADDR + db)),
            ins(f"ds_read_b64_tr_b16 {v(f + 2, 2)}, {v(TADDR + 4 + db)} offset:{off}", "ds", dst=v(f + 2, 2),
                src=v(TADDR + 4 + db))]


def dma(i, dmabuf):
    """copy instruction i of a block (0, 1: K rows; 2, 3: V rows) into buffer dmabuf"""
    kv = i // 2
    base = (0 if kv == 0 else 65536) + dmabuf * 8192 + (i % 2) * 1024
    desc = s(DK, 4) if kv == 0 else s(DV, 4)
    return [ins(f"s_add_u32 m0, %[dbase], {base}", "m0", dst=["m0"]),
            ins(f"buffer_load_dwordx4 {v(DOFF + i % 2)}, {desc}, 0 offen lds", "vmem", src=[v(DOFF + i % 2), "m0"])]


def valu(par, gate):
    sv = lambda qg, r: v(S[par] + 16 * qg + r)
    dv = lambda qg, r: v(DP[par] + 16 * qg + r)
    order = [(qg, r) for r in range(16) for qg in range(2)]
    fma = {e: ins(f"v_fma_f32 {sv(*e)}, {sv(*e)}, %[c2], -{v(LSE + e[0])}", "valu", dst=sv(*e),
                  src=f"{sv(*e)} {v(LSE + e[0])}") for e in order}
    ex = {e: ins(f"v_exp_f32_e64 {sv(*e)}, {sv(*e)} clamp", "trans", dst=sv(*e), src=sv(*e)) for e in order}
    mul = {e: ins(f"v_mul_f32_e32 {dv(*e)}, {sv(*e)}, {dv(*e)}", "valu", dst=dv(*e), src=f"{sv(*e)} {dv(*e)}")
           for e in order}
    cvt = []
    for qg in range(2):
        for r in range(1, 16, 2):
            k2, j = r // 8, (r - 1) % 8
            dst = v(DS + qg * 8 + k2 * 4 + j // 2)
            c = ins(f"v_cvt_pk_bf16_f32 {dst}, {dv(qg, r - 1)}, {dv(qg, r)}", "valu", dst=dst,
                    src=f"{dv(qg, r - 1)} {dv(qg, r)}")
            c.not_before = gate
            cvt.append((r, qg, c))
    L = []
    n = len(order)
    for k in range(n + 8):  # skewed: fma(k), exp(k - 2), mul(k - 4)
        if k < n:
            L.append(fma[order[k]])
        if 0 <= k - 2 < n:
            L.append(ex[order[k - 2]])
        if 0 <= k - 4 < n:
            L.append(mul[order[k - 4]])
    L += [c for _, _, c in sorted(cvt)]  # after the dQ MFMAs that read the previous dS^T
    return L


PAIRS = ["Q0", "Q1", "Q2", "S0", "Q3", "P0", "Q4", "S1", "Q5", "P1", "Q6", "S2", "Q7", "P2", "S3", "P3", "S4",
         "P4", "S5", "P5", "S6", "P6", "S7", "P7"]
DMA_AT = (1, 13, 25, 37)
BUDGET = 20


def slot_body(u, entry):
    par, kbuf, tbuf, tnext, dmabuf = u % 2, (u + 1) % 8, (u + 7) % 8, u, (u + 5) % 8
    em = Emitter.merged_entry(entry)
    mf, idx, pinned = [], {}, {}
    for p in PAIRS:
        idx[p] = len(mf)
        k = int(p[1])
        mf += mf_dq(k) if p[0] == "Q" else (mf_s(k, par) if p[0] == "S" else mf_dp(k, par))
    koff = kbuf * 8192  # V addresses carry the 64 KiB region base
    pinned[0] = ds_t(2, tbuf) + ds_t(3, tbuf) + ds_row(KADDR, KF, 0, koff) + ds_row(KADDR, KF, 1, koff)
    pinned.setdefault(2, []).extend(ds_row(VADDR, VF, 0, koff) + ds_row(VADDR, VF, 1, koff))
    pinned.setdefault(4, []).extend(ds_row(KADDR, KF, 2, koff) + ds_row(VADDR, VF, 2, koff))
    pinned.setdefault(6, []).extend(ds_row(KADDR, KF, 3, koff) + ds_row(VADDR, VF, 3, koff))
    for ks in range(4, 8):
        pinned.setdefault(idx[f"S{ks - 4}"] + 2, []).extend(ds_row(KADDR, KF, ks, koff))
        pinned.setdefault(idx[f"P{ks - 4}"] + 2, []).extend(ds_row(VADDR, VF, ks, koff))
    for i in range(4, 8):
        pinned.setdefault(idx[f"Q{i - 4}"] + 2, []).extend(ds_t(i, tbuf))
    pinned.setdefault(idx["Q4"] + 2, []).extend(ds_t(0, tnext))  # the next slot's first two K^T fragments
    pinned.setdefault(idx["Q5"] + 2, []).extend(ds_t(1, tnext))
    for i, at in enumerate(DMA_AT):
        pinned.setdefault(at, []).extend(dma(i, dmabuf))
    left = fill_schedule(em, mf, valu(par, idx["Q7"] + 2), budget=BUDGET, pinned=pinned)
    em.emit_all(left)
    return em


def prologue():
    em = Emitter()
    for r in range(KF, DS + 16):  # fragments and dS(-1) = 0
        em.raw(f"v_mov_b32 {v(r)}, 0", 1)
    for r in range(128):
        em.raw(f"v_accvgpr_write_b32 {a(r)}, 0", 1)
    em.raw("s_cmp_eq_u32 %[nb], 0")
    em.raw(f"s_cbranch_scc1 {lbl('done')}")
    em.raw("s_waitcnt lgkmcnt(0)")  # the zero fill of K buffer 7 (dQ(-1) reads it with dS = 0)
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
    for ks in range(8):  # S^T(0), dP^T(0) into S[0], DP[0] (slot 0 has par 0)
        mf += mf_s(ks, 1) + mf_dp(ks, 1)
    pinned = {0: ds_row(KADDR, KF, 0, 0) + ds_row(KADDR, KF, 1, 0) + ds_row(VADDR, VF, 0, 0) + ds_row(VADDR, VF, 1, 0)}
    for ks in range(2, 8):
        pinned.setdefault(4 * (ks - 2) + 2, []).extend(ds_row(KADDR, KF, ks, 0) + ds_row(VADDR, VF, ks, 0))
    pinned.setdefault(28, []).extend(ds_t(0, 7) + ds_t(1, 7))  # slot 0's dQ(-1) fragments (zeros)
    fill_schedule(em, mf, [], pinned=pinned)
    return em


def final_dq(u, entry):
    """dQ(NB-1) after the last slot (J = NB - 1, J % 8 == u): dS^T just
    written, K^T from buffer u; its first two fragments were prefetched."""
    em = Emitter.merged_entry(entry)
    mf = []
    pinned = {0: ds_t(2, u) + ds_t(3, u)}
    for i in range(8):
        mf += mf_dq(i)
    for i in range(4, 8):
        pinned[2 * (i - 4) + 2] = ds_t(i, u)
    fill_schedule(em, mf, [], pinned=pinned)
    em.settle()
    return em


def build():
    """The loop's lines."""
    pro = prologue()
    bodies, ends = {}, {u: [] for u in range(8)}
    for _ in range(4):
        new = {}
        for u in range(8):
            prev = ends[(u - 1) % 8] + ([pro] if u == 0 else [])
            new[u] = slot_body(u, prev or [pro])
        bodies = new
        ends = {u: [bodies[u]] for u in range(8)}
    lines = list(pro.lines)
    lines.append(f"{lbl('loop')}:")
    for u in range(8):
        if u % 2 == 0:
            lines += ["s_waitcnt vmcnt(8)", "s_barrier"]
        lines += cursor_desc((u + 5) % 8)
        lines += bodies[u].lines
        lines += cursor_adv(f"s{u}")
        lines.append(f"s_add_u32 {s(J)}, {s(J)}, 1")
        lines.append(f"s_cmp_eq_u32 {s(J)}, %[nb]")
        lines.append(f"s_cbranch_scc1 {lbl(f'exit{u}')}")
    lines.append(f"s_branch {lbl('loop')}")
    for u in range(8):
        lines.append(f"{lbl(f'exit{u}')}:")
        lines += final_dq(u, [bodies[u]]).lines
        lines.append(f"s_branch {lbl('done')}")
    lines.append(f"{lbl('done')}:")
    lines.append("s_waitcnt vmcnt(0) lgkmcnt(0)")
    return lines


def render(lines):
    def body(ls):
        return " \\\n".join('  "' + ln + '\\n\\t"' for ln in ls)
    return ("// Generated by dq_asm_gen.py: the main loop of dq_asm_kernel (dq_asm.hip).\n"
            "// Do not edit; change the generator and rebuild.\n"
            "#pragma once\n"
            f"#define HARP_DQ_ASM_SGPR_CLOBBERS {clobber_list(SGPR_CLOBBER)}\n"
            f"#define HARP_DQ_ASM_LOOP \\\n{body(lines)}\n")


def write(path=None):
    path = path or os.path.join(os.path.dirname(os.path.abspath(__file__)), "dq_asm.inc")
    text = render(build())
    old = open(path).read() if os.path.exists(path) else None
    if old != text:
        with open(path, "w") as f:
            f.write(text)
    return path


if __name__ == "__main__":
    p = write()
    print(p, sum(1 for _ in open(p)), "lines")
