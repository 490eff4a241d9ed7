"""CPU model of the generated dK/dV loop (harp_amd/csrc/dkdv_asm_gen.py, the
loop of dkdv_asm_kernel) for one block of 4 waves, with the kernel's set-up
and epilogue (dkdv_asm.hip) restated in Python.

Test infrastructure: it executes the generator's instruction list with the
documented semantics of each gfx950 instruction it uses
(v_mfma_f32_32x32x16_bf16 operand / accumulator layouts, ds_read_b64_tr_b16's
lane mapping, buffer_load ... lds, the VALU and SALU subset), so the CPU tests
check the loop's data layout, operand roles, buffer rotation and carried
work without a GPU.  Timing is not modelled: copies land when issued and the
waves run in lockstep between barriers, so wait counts and hazards are the
GPU tests' business."""
import re
import sys

import numpy as np

sys.path.insert(0, str(__import__('pathlib').Path(__file__).resolve().parents[1] / 'harp_amd' / 'csrc'))
import dkdv_asm_gen as G  # noqa: E402

LDS_BYTES = 163840
KBUF = 16384
KV_OFF = 5 * KBUF
VROW = 272
ST_OFF = KV_OFF + 256 * VROW
ST_PER_WAVE = 5 * 512


def swz(r):
    return ((r & 3) << 2) | ((r >> 2) & 3)


def f2bf(x):
    """fp32 array -> bf16 bits (round to nearest even)"""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7fff + ((u >> 16) & 1)) >> 16) & 0xffff
    return r.astype(np.uint32)


def bf2f(b):
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


class Mem:
    """global memory: named byte buffers at fake 48-bit addresses"""

    def __init__(self):
        self.bufs = []
        self.next = 0x100000000

    def add(self, arr):
        b = np.frombuffer(np.ascontiguousarray(arr).tobytes(), dtype=np.uint8).copy()
        base = self.next
        self.bufs.append((base, b))
        self.next += (len(b) + 0xfffff) & ~0xfffff
        self.next += 0x100000
        return base

    def read(self, addr, n):
        for base, b in self.bufs:
            if base <= addr and addr + n <= base + len(b):
                return b[addr - base:addr - base + n]
        raise RuntimeError(f"global read out of any buffer: {addr:#x} + {n}")


class Wave:
    def __init__(self, w):
        self.w = w
        self.v = np.zeros((256, 64), dtype=np.uint32)
        self.a = np.zeros((256, 64), dtype=np.uint32)
        self.s = {}
        self.m0 = 0
        self.scc = 0


REG = re.compile(r"^([vas])\[(\d+):(\d+)\]$|^([vas])(\d+)$")


def reg(tok):
    m = REG.match(tok)
    if not m:
        return None
    if m.group(1):
        return m.group(1), int(m.group(2)), int(m.group(3)) - int(m.group(2)) + 1
    return m.group(4), int(m.group(5)), 1


class Emu:
    def __init__(self, lines, ops, mem, lds):
        self.lines = [ln for ln in lines]
        self.ops = ops
        self.mem = mem
        self.lds = lds
        self.labels = {ln[:-1]: i for i, ln in enumerate(self.lines) if ln.endswith(':')}
        self.count = {}

    def sval(self, wv, tok):
        """scalar operand value (uint32 or uint64 for pairs)"""
        tok = tok.strip()
        if tok.startswith('%['):
            return self.ops[tok[2:-1]]
        r = reg(tok)
        if r and r[0] == 's':
            k, i, n = r
            if n == 1:
                return wv.s.get(i, 0)
            return wv.s.get(i, 0) | (wv.s.get(i + 1, 0) << 32)
        if tok == 'm0':
            return wv.m0
        return int(tok, 0)

    def vsrc(self, wv, tok):
        tok = tok.strip()
        r = reg(tok)
        if r and r[0] == 'v':
            return wv.v[r[1]].copy()
        if r and r[0] == 'a':
            return wv.a[r[1]].copy()
        if r and r[0] == 's':
            return np.full(64, self.sval(wv, tok) & 0xffffffff, dtype=np.uint32)
        if tok.startswith('%['):
            val = self.ops[tok[2:-1]]
            if isinstance(val, float):
                return np.full(64, np.float32(val).view(np.uint32), dtype=np.uint32)
            return np.full(64, val & 0xffffffff, dtype=np.uint32)
        if tok in ('0', '1.0'):
            return np.full(64, 0 if tok == '0' else 0x3f800000, dtype=np.uint32)
        return np.full(64, int(tok, 0) & 0xffffffff, dtype=np.uint32)

    def regfile(self, wv, k):
        return wv.v if k == 'v' else wv.a

    def tup(self, wv, tok):
        k, i, n = reg(tok)
        return self.regfile(wv, k)[i:i + n]

    def step(self, wv, pc):
        """execute line pc of wave wv; return next pc, or ('barrier', pc+1) / None at end"""
        ln = self.lines[pc]
        if ln.endswith(':') or not ln:
            return pc + 1
        op, _, rest = ln.partition(' ')
        args = [x.strip() for x in rest.split(',')] if rest else []
        self.count[op] = self.count.get(op, 0) + 1
        if op in ('s_nop', 's_waitcnt'):
            return pc + 1
        if op == 's_barrier':
            return ('barrier', pc + 1)
        if op == 's_branch':
            return self.labels[args[0]]
        if op == 's_cbranch_scc1':
            return self.labels[args[0]] if wv.scc else pc + 1
        if op == 's_cmp_eq_u32':
            wv.scc = int((self.sval(wv, args[0]) & 0xffffffff) == (self.sval(wv, args[1]) & 0xffffffff))
            return pc + 1
        if op == 's_mov_b32':
            wv.s[reg(args[0])[1]] = self.sval(wv, args[1]) & 0xffffffff
            return pc + 1
        if op == 's_mov_b64':
            x = self.sval(wv, args[1])
            i = reg(args[0])[1]
            wv.s[i], wv.s[i + 1] = x & 0xffffffff, (x >> 32) & 0xffffffff
            return pc + 1
        if op == 's_add_u32':
            x = (self.sval(wv, args[1]) & 0xffffffff) + (self.sval(wv, args[2]) & 0xffffffff)
            wv.scc = int(x >> 32)
            if args[0] == 'm0':
                wv.m0 = x & 0xffffffff
            else:
                wv.s[reg(args[0])[1]] = x & 0xffffffff
            return pc + 1
        if op == 's_addc_u32':
            x = (self.sval(wv, args[1]) & 0xffffffff) + (self.sval(wv, args[2]) & 0xffffffff) + wv.scc
            wv.scc = int(x >> 32)
            wv.s[reg(args[0])[1]] = x & 0xffffffff
            return pc + 1
        if op == 's_sub_i32':
            a_, b_ = self.sval(wv, args[1]) & 0xffffffff, self.sval(wv, args[2]) & 0xffffffff
            a_ = a_ - (1 << 32) if a_ >> 31 else a_
            b_ = b_ - (1 << 32) if b_ >> 31 else b_
            wv.s[reg(args[0])[1]] = (a_ - b_) & 0xffffffff
            return pc + 1
        if op == 's_max_i32':
            a_, b_ = self.sval(wv, args[1]) & 0xffffffff, self.sval(wv, args[2]) & 0xffffffff
            a_ = a_ - (1 << 32) if a_ >> 31 else a_
            b_ = b_ - (1 << 32) if b_ >> 31 else b_
            wv.s[reg(args[0])[1]] = max(a_, b_) & 0xffffffff
            return pc + 1
        if op == 'v_mov_b32':
            wv.v[reg(args[0])[1]] = self.vsrc(wv, args[1])
            return pc + 1
        if op == 'v_accvgpr_write_b32':
            wv.a[reg(args[0])[1]] = self.vsrc(wv, args[1])
            return pc + 1
        if op == 'v_add_u32_e32':
            wv.v[reg(args[0])[1]] = (self.vsrc(wv, args[1]).astype(np.uint64) +
                                     self.vsrc(wv, args[2]).astype(np.uint64)).astype(np.uint32)
            return pc + 1
        if op == 'v_mul_f32_e32':
            x = self.vsrc(wv, args[1]).view(np.float32) * self.vsrc(wv, args[2]).view(np.float32)
            wv.v[reg(args[0])[1]] = x.astype(np.float32).view(np.uint32)
            return pc + 1
        if op == 'v_exp_f32_e64':
            src = args[1].split()[0]
            x = np.exp2(self.vsrc(wv, src).view(np.float32).astype(np.float64))
            if 'clamp' in args[1]:
                x = np.clip(x, 0.0, 1.0)
            wv.v[reg(args[0])[1]] = x.astype(np.float32).view(np.uint32)
            return pc + 1
        if op == 'v_cvt_pk_bf16_f32':
            lo = f2bf(self.vsrc(wv, args[1]).view(np.float32))
            hi = f2bf(self.vsrc(wv, args[2]).view(np.float32))
            wv.v[reg(args[0])[1]] = lo | (hi << 16)
            return pc + 1
        if op in ('buffer_load_dwordx4', 'buffer_load_dword'):
            voff = self.vsrc(wv, args[0])
            k, si, _ = reg(args[1].strip())
            base = wv.s[si] | ((wv.s[si + 1] & 0xffff) << 32)
            nrec = wv.s[si + 2]
            size = 16 if op.endswith('x4') else 4
            for lane in range(64):
                o = int(voff[lane])
                dst = wv.m0 + lane * size
                if o + size <= nrec:
                    data = self.mem.read(base + o, size)
                else:
                    data = np.zeros(size, dtype=np.uint8)
                if dst + size > LDS_BYTES:
                    raise RuntimeError(f"LDS DMA out of range {dst}")
                self.lds[dst:dst + size] = data
            return pc + 1
        if op == 'ds_read_b128':
            at, offt = args[1].split()
            addr = self.vsrc(wv, at).astype(np.int64) + int(offt.split(':')[1])
            dst = reg(args[0])
            out = np.zeros((4, 64), dtype=np.uint32)
            for lane in range(64):
                ad = int(addr[lane])
                if ad + 16 > LDS_BYTES:
                    raise RuntimeError(f"LDS read out of range {ad}")
                out[:, lane] = self.lds[ad:ad + 16].view(np.uint32)
            wv.v[dst[1]:dst[1] + 4] = out
            return pc + 1
        if op == 'ds_read_b64_tr_b16':
            at, offt = args[1].split()
            addr = self.vsrc(wv, at).astype(np.int64) + int(offt.split(':')[1])
            dst = reg(args[0])
            half = np.zeros((4, 64), dtype=np.uint32)  # 4 x 16-bit slots
            for lane in range(64):
                grp, i = lane // 16, lane % 16
                for sl in range(4):
                    src_lane = 16 * grp + 4 * sl + i // 4
                    ad = int(addr[src_lane])
                    if ad + 8 > LDS_BYTES:
                        raise RuntimeError(f"LDS tr read out of range {ad}")
                    h = self.lds[ad:ad + 8].view(np.uint16)[i % 4]
                    half[sl, lane] = h
            wv.v[dst[1]] = half[0] | (half[1] << 16)
            wv.v[dst[1] + 1] = half[2] | (half[3] << 16)
            return pc + 1
        if op == 'v_mfma_f32_32x32x16_bf16':
            D = reg(args[0])
            A = self.tup(wv, args[1])
            B = self.tup(wv, args[2])
            if args[3] == '0':
                C = np.zeros((16, 64), dtype=np.uint32)
            else:
                C = self.tup(wv, args[3]).copy()
            # unpack A[m][k]: lane l: m = l % 32, k = 8 (l // 32) + j
            def unpack(T):
                e = np.zeros((8, 64), dtype=np.float32)
                for j in range(4):
                    e[2 * j] = bf2f(T[j] & 0xffff)
                    e[2 * j + 1] = bf2f(T[j] >> 16)
                return e
            ea, eb = unpack(A), unpack(B)
            Am = np.zeros((32, 16), dtype=np.float64)
            Bm = np.zeros((16, 32), dtype=np.float64)
            for l in range(64):
                for j in range(8):
                    Am[l % 32, 8 * (l // 32) + j] = ea[j, l]
                    Bm[8 * (l // 32) + j, l % 32] = eb[j, l]
            Cm = np.zeros((32, 32), dtype=np.float64)
            cf = C.view(np.float32)
            for l in range(64):
                for r in range(16):
                    Cm[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32] = cf[r, l]
            Dm = Am @ Bm + Cm
            out = np.zeros((16, 64), dtype=np.float32)
            for l in range(64):
                for r in range(16):
                    out[r, l] = Dm[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32]
            self.regfile(wv, D[0])[D[1]:D[1] + 16] = out.view(np.uint32)
            return pc + 1
        raise NotImplementedError(ln)

    def run(self, waves, max_steps=10 ** 8):
        pcs = [0] * len(waves)
        done = [False] * len(waves)
        steps = 0
        while not all(done):
            for wi, wv in enumerate(waves):
                if done[wi]:
                    continue
                while True:
                    if pcs[wi] >= len(self.lines):
                        done[wi] = True
                        break
                    r = self.step(wv, pcs[wi])
                    steps += 1
                    if steps > max_steps:
                        raise RuntimeError("too many steps")
                    if isinstance(r, tuple):
                        pcs[wi] = r[1]
                        break
                    pcs[wi] = r


def run_block(q, k, v, do, stats0, stats1, scale, len_valid, kblk0=0):
    """q, do [T, 128] bf16 bits (uint16); k, v [rows, 128] bf16 bits; stats planes [T] fp32.
    Returns dK, dV [256, 128] of the block (fp32, dK scaled, pads 0)."""
    T = q.shape[0]
    mem = Mem()
    qa = mem.add(q.astype(np.uint16))
    ga = mem.add(do.astype(np.uint16))
    s0a = mem.add(stats0.astype(np.float32))
    s1a = mem.add(stats1.astype(np.float32))
    lds = np.zeros(LDS_BYTES, dtype=np.uint8)
    # V tile
    for row in range(256):
        key = kblk0 + row
        if key < len_valid:
            lds[KV_OFF + row * VROW:KV_OFF + row * VROW + 256] = np.frombuffer(v[key].astype(np.uint16).tobytes(),
                                                                             dtype=np.uint8)
    qrow = 256
    c2 = np.float32(scale * 1.4426950408889634)
    nb = (T + 31) // 32 if kblk0 < len_valid else 0
    waves = []
    for w in range(4):
        wv = Wave(w)
        lane = np.arange(64)
        l32, g = lane & 31, lane >> 5
        mv = np.zeros((32, 64), dtype=np.int64)
        for ks in range(8):
            mv[ks] = l32 * 256 + (((2 * ks + g) ^ np.vectorize(swz)(l32)) << 4)
        j, sr, m = lane >> 4, (lane >> 2) & 3, lane & 3
        cl = 2 * (j & 1) + (m >> 1)
        for hh in range(2):
            for db in range(4):
                row = 8 * hh + 4 * g + sr
                mv[8 + hh * 4 + db] = 4 * KBUF + 2 * (row * 128 + (((4 * db + cl) ^ np.vectorize(swz)(row)) << 3)
                                                      + 4 * (m & 1))
        mv[16] = KV_OFF + (w * 64 + l32) * VROW + g * 16
        mv[17] = ST_OFF + w * ST_PER_WAVE + g * 16
        for i in range(2):
            r = (2 * w + i) * 4 + (lane >> 4)
            chunk = ((lane & 15) ^ np.vectorize(swz)(r)) << 4
            mv[18 + i] = r * qrow + chunk
            mv[20 + i] = r * qrow + chunk
        mv[22] = lane * 4
        for i in range(23, 32):
            mv[i] = mv[16]
        wv.v[0:32] = mv.astype(np.uint32)
        # K B operands
        for kg in range(2):
            for ks in range(8):
                for ln in range(64):
                    key = kblk0 + w * 64 + kg * 32 + (ln & 31)
                    gg = ln >> 5
                    if key < len_valid:
                        e = k[key, ks * 16 + gg * 8: ks * 16 + gg * 8 + 8].astype(np.uint32)
                    else:
                        e = np.zeros(8, dtype=np.uint32)
                    for jj in range(4):
                        wv.v[32 + kg * 32 + ks * 4 + jj, ln] = e[2 * jj] | (e[2 * jj + 1] << 16)
        waves.append(wv)
    ops_common = dict(c2=float(c2), qp=qa, gp=ga, sp0=s0a, sp1=s1a, qnr=T * qrow, gnr=T * qrow, snr=T * 4,
                      qstep=32 * qrow, gstep=32 * qrow, nb=nb)
    lines = [ln.replace('%=', '0') for ln in G.build()]
    # per-wave operands differ (dbase, sbase): run with a wave-indexed ops table
    emus = []
    for w in range(4):
        ops = dict(ops_common, dbase=w * 2048, sbase=ST_OFF + w * ST_PER_WAVE)
        emus.append(Emu(lines, ops, mem, lds))
    # lockstep between barriers
    pcs = [0] * 4
    done = [False] * 4
    while not all(done):
        for w in range(4):
            if done[w]:
                continue
            while True:
                if pcs[w] >= len(lines):
                    done[w] = True
                    break
                r = emus[w].step(waves[w], pcs[w])
                if isinstance(r, tuple):
                    pcs[w] = r[1]
                    break
                pcs[w] = r
    dk = np.zeros((256, 128), dtype=np.float64)
    dv = np.zeros((256, 128), dtype=np.float64)
    for w in range(4):
        af = waves[w].a.view(np.float32)
        for kg in range(2):
            for db in range(4):
                for r in range(16):
                    for ln in range(64):
                        key = w * 64 + kg * 32 + 8 * (r // 4) + 4 * (ln >> 5) + r % 4
                        d = db * 32 + (ln & 31)
                        valid = kblk0 + key < len_valid
                        dk[key, d] = af[64 * kg + 16 * db + r, ln] * scale if valid else 0.0
                        dv[key, d] = af[128 + 64 * kg + 16 * db + r, ln] if valid else 0.0
    return dk, dv, waves


def reference(q, k, v, do, scale, len_valid):
    """fp64 dK, dV for one chunk (keys [0, len_valid)), all T queries"""
    Q, K, V, dO = (bf2f(x.astype(np.uint32)).astype(np.float64) for x in (q, k, v, do))
    K, V = K[:len_valid], V[:len_valid]
    S = Q @ K.T * scale
    m = S.max(axis=1, keepdims=True)
    P = np.exp(S - m)
    lsum = P.sum(axis=1, keepdims=True)
    P = P / lsum
    O = P @ V
    Dl = (dO * O).sum(axis=1, keepdims=True)
    dP = dO @ V.T
    dS = P * (dP - Dl)
    dK = dS.T @ Q * scale
    dV = P.T @ dO
    lse = (m + np.log(lsum))[:, 0]
    return dK, dV, lse, Dl[:, 0]
