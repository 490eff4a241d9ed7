"""CPU model of the generated hand-scheduled loops (harp_amd/csrc/
dkdv_asm_gen.py, dq_asm_gen.py, fwd_asm_gen.py: the loops of dkdv_asm_kernel,
dq_asm_kernel and fwd_asm_kernel) for one block of 4 waves, with each
kernel's set-up and epilogue (dkdv_asm.hip, dq_asm.hip, fwd_asm.hip) restated
in Python; the dQ and forward loops read a chunk table from a modelled
kernarg block, so their scalar copy cursor runs as on the GPU.

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
        self.vcc = np.zeros(64, dtype=bool)


REG = re.compile(r"^([vas])\[(\d+):(\d+)\]$|^([vas])(\d+)$")


def reg(tok):
    m = REG.match(tok)
    if not m:
        return None
    if m.group(1):
        return m.group(1), int(m.group(2)), int(m.group(3)) - int(m.group(2)) + 1
    return m.group(4), int(m.group(5)), 1


_LANE = np.arange(64)
_ROW_AB = _LANE % 32                                   # A: row m; B: column n
_K_AB = 8 * (_LANE // 32)[None, :] + np.arange(8)[:, None]   # k of element j of lane l
_R = np.arange(16)
_ROW_C = (8 * (_R // 4))[:, None] + 4 * (_LANE // 32)[None, :] + (_R % 4)[:, None]  # C row of (reg r, lane l)


def _unpack(T):
    e = np.zeros((8, 64), dtype=np.float32)
    e[0::2] = bf2f(T & 0xffff)
    e[1::2] = bf2f(T >> 16)
    return e


def mfma_32x32x16(A, B, C):
    """v_mfma_f32_32x32x16_bf16: A lane l holds A[l % 32][8 (l / 32) + j], B
    lane l holds B[8 (l / 32) + j][l % 32] (j = 0..7, low half first), C / D
    register r of lane l is row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32."""
    Am = np.zeros((32, 16), dtype=np.float64)
    Bm = np.zeros((16, 32), dtype=np.float64)
    Am[_ROW_AB[None, :], _K_AB] = _unpack(A)
    Bm[_K_AB, _ROW_AB[None, :]] = _unpack(B)
    Cm = np.zeros((32, 32), dtype=np.float64)
    Cm[_ROW_C, np.broadcast_to(_ROW_AB, (16, 64))] = C.view(np.float32)
    Dm = Am @ Bm + Cm
    return Dm[_ROW_C, np.broadcast_to(_ROW_AB, (16, 64))].astype(np.float32).view(np.uint32)


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
        if tok == 'vcc':
            return sum(1 << l for l in range(64) if wv.vcc[l])
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
            C = np.zeros((16, 64), dtype=np.uint32) if args[3] == '0' else self.tup(wv, args[3]).copy()
            self.regfile(wv, D[0])[D[1]:D[1] + 16] = mfma_32x32x16(A, B, C)
            return pc + 1
        return self.step_more(wv, pc, op, args, ln)

    # ---- the rest of the subset (dQ and forward loops) ----------------------
    def mask(self, wv, tok):
        tok = tok.strip()
        if tok == 'vcc':
            return wv.vcc.copy()
        k, i, n = reg(tok)
        x = wv.s.get(i, 0) | (wv.s.get(i + 1, 0) << 32)
        return np.array([(x >> l) & 1 for l in range(64)], dtype=bool)

    def set_mask(self, wv, tok, m):
        if tok == 'vcc':
            wv.vcc = m.copy()
            return
        x = 0
        for l in range(64):
            if m[l]:
                x |= 1 << l
        i = reg(tok)[1]
        wv.s[i], wv.s[i + 1] = x & 0xffffffff, x >> 32

    def fsrc(self, wv, tok):
        tok = tok.strip()
        neg = tok.startswith('-')
        if neg:
            tok = tok[1:]
        if tok == '1.0':
            x = np.full(64, 1.0, dtype=np.float32)
        else:
            x = self.vsrc(wv, tok).view(np.float32).copy()
        return -x if neg else x

    @staticmethod
    def i32(x):
        x &= 0xffffffff
        return x - (1 << 32) if x >> 31 else x

    def step_more(self, wv, pc, op, args, ln):
        S = lambda t: self.sval(wv, t) & 0xffffffff
        def setd(val):
            wv.s[reg(args[0])[1]] = val & 0xffffffff
        if op == 's_add_i32':
            setd(self.i32(S(args[1])) + self.i32(S(args[2])))
        elif op == 's_and_b32':
            setd(S(args[1]) & S(args[2]))
            wv.scc = int((S(args[1]) & S(args[2])) != 0)
        elif op == 's_or_b32':
            setd(S(args[1]) | S(args[2]))
            wv.scc = int((S(args[1]) | S(args[2])) != 0)
        elif op == 's_lshl_b32':
            setd(S(args[1]) << (S(args[2]) & 31))
        elif op == 's_mul_i32':
            setd(self.i32(S(args[1])) * self.i32(S(args[2])))
        elif op == 's_min_u32':
            setd(min(S(args[1]), S(args[2])))
        elif op == 's_bfe_u32':
            src1 = S(args[2])
            off, width = src1 & 31, (src1 >> 16) & 0x7f
            setd((S(args[1]) >> off) & ((1 << width) - 1))
        elif op in ('s_cmp_ge_i32', 's_cmp_gt_i32', 's_cmp_le_i32'):
            a_, b_ = self.i32(S(args[0])), self.i32(S(args[1]))
            wv.scc = int({'s_cmp_ge_i32': a_ >= b_, 's_cmp_gt_i32': a_ > b_, 's_cmp_le_i32': a_ <= b_}[op])
        elif op == 's_cmp_lt_u32':
            wv.scc = int(S(args[0]) < S(args[1]))
        elif op == 's_cmp_lg_u64':
            wv.scc = int(self.sval(wv, args[0]) != self.sval(wv, args[1]))
        elif op == 's_or_b64':
            x = self.sval(wv, args[1]) | self.sval(wv, args[2])
            i = reg(args[0])[1]
            wv.s[i], wv.s[i + 1] = x & 0xffffffff, (x >> 32) & 0xffffffff
            wv.scc = int(x != 0)
        elif op in ('s_load_dword', 's_load_dwordx2'):
            addr = self.sval(wv, args[1]) + S(args[2])
            n = 4 if op == 's_load_dword' else 8
            data = self.mem.read(addr, n).view(np.uint32)
            i = reg(args[0])[1]
            for j in range(n // 4):
                wv.s[i + j] = int(data[j])
        elif op == 'v_mov_b32_e32':
            wv.v[reg(args[0])[1]] = self.vsrc(wv, args[1])
        elif op == 'v_accvgpr_read_b32':
            wv.v[reg(args[0])[1]] = wv.a[reg(args[1])[1]].copy()
        elif op == 'v_fma_f32':
            x = (self.fsrc(wv, args[1]).astype(np.float64) * self.fsrc(wv, args[2]) + self.fsrc(wv, args[3]))
            wv.v[reg(args[0])[1]] = x.astype(np.float32).view(np.uint32)
        elif op == 'v_exp_f32_e32':
            with np.errstate(over='ignore'):  # exps that overflow to inf, as the hardware's do
                x = np.exp2(self.fsrc(wv, args[1]).astype(np.float64))
            wv.v[reg(args[0])[1]] = x.astype(np.float32).view(np.uint32)
        elif op in ('v_add_f32_e32', 'v_sub_f32_e32', 'v_max_f32_e32'):
            a_, b_ = self.fsrc(wv, args[1]), self.fsrc(wv, args[2])
            x = a_ + b_ if op == 'v_add_f32_e32' else (a_ - b_ if op == 'v_sub_f32_e32' else np.maximum(a_, b_))
            wv.v[reg(args[0])[1]] = x.astype(np.float32).view(np.uint32)
        elif op == 'v_max3_f32':
            x = np.maximum(np.maximum(self.fsrc(wv, args[1]), self.fsrc(wv, args[2])), self.fsrc(wv, args[3]))
            wv.v[reg(args[0])[1]] = x.astype(np.float32).view(np.uint32)
        elif op == 'v_sub_u32_e32':
            wv.v[reg(args[0])[1]] = (self.vsrc(wv, args[1]).astype(np.int64) -
                                     self.vsrc(wv, args[2]).astype(np.int64)).astype(np.uint32)
        elif op in ('v_cmp_gt_f32_e64', 'v_cmp_eq_f32_e64', 'v_cmp_lt_f32_e32'):
            a_, b_ = self.fsrc(wv, args[1]), self.fsrc(wv, args[2])
            m = {'v_cmp_gt_f32_e64': a_ > b_, 'v_cmp_eq_f32_e64': a_ == b_, 'v_cmp_lt_f32_e32': a_ < b_}[op]
            self.set_mask(wv, args[0], m)
        elif op == 'v_cmp_ge_i32_e32':
            a_ = self.vsrc(wv, args[1]).view(np.int32)
            b_ = self.vsrc(wv, args[2]).view(np.int32)
            self.set_mask(wv, args[0], a_ >= b_)
        elif op in ('v_cndmask_b32_e32', 'v_cndmask_b32_e64'):
            m = self.mask(wv, args[3])
            a_ = self.fsrc(wv, args[1]).view(np.uint32)
            b_ = self.fsrc(wv, args[2]).view(np.uint32)
            wv.v[reg(args[0])[1]] = np.where(m, b_, a_)
        elif op == 'v_permlane32_swap_b32_e32':
            i, j = reg(args[0])[1], reg(args[1])[1]
            t = wv.v[i, 32:].copy()
            wv.v[i, 32:] = wv.v[j, :32]
            wv.v[j, :32] = t
        else:
            raise NotImplementedError(ln)
        return pc + 1

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
                mv[8 + hh * 4 + db] = G.TADDR_BUF0 * KBUF + 2 * (row * 128 + (((4 * db + cl) ^ np.vectorize(swz)(row))
                                                                 << 3) + 4 * (m & 1))
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


# ---- the dQ and forward loops (dq_asm.hip, fwd_asm.hip) ------------------
import dq_asm_gen as GQ  # noqa: E402
import fwd_asm_gen as GF  # noqa: E402

OOFF, LOFF, KOFF, VOFF = 0, 64, 128, 256   # chunk-table fields in the modelled kernarg block


LAST_COUNTS = {}  # opcode -> executions, summed over the waves of the last dQ / forward run


def _lockstep(lines, ops_per_wave, mem, lds, waves):
    emus = [Emu(lines, ops, mem, lds) for ops in ops_per_wave]
    pcs = [0] * len(waves)
    done = [False] * len(waves)
    while not all(done):
        for w in range(len(waves)):
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
    LAST_COUNTS.clear()
    for e in emus:
        for k, n in e.count.items():
            LAST_COUNTS[k] = LAST_COUNTS.get(k, 0) + n


def _chunk_setup(mem, ks, vs, lens, order):
    """chunk K / V buffers ([rows, 128] bf16 bits) and the kernarg block with
    order, len, k, v at OOFF / LOFF / KOFF / VOFF"""
    kad = [mem.add(k.astype(np.uint16)) for k in ks]
    vad = [mem.add(v.astype(np.uint16)) for v in vs]
    karg = np.zeros(512, dtype=np.uint8)
    karg[OOFF:OOFF + 4 * len(order)] = np.frombuffer(np.array(order, dtype=np.int32).tobytes(), dtype=np.uint8)
    karg[LOFF:LOFF + 4 * len(lens)] = np.frombuffer(np.array(lens, dtype=np.int32).tobytes(), dtype=np.uint8)
    karg[KOFF:KOFF + 8 * len(kad)] = np.frombuffer(np.array(kad, dtype=np.uint64).tobytes(), dtype=np.uint8)
    karg[VOFF:VOFF + 8 * len(vad)] = np.frombuffer(np.array(vad, dtype=np.uint64).tobytes(), dtype=np.uint8)
    ctp = mem.add(karg)
    # the cursor's first chunk (kv_enter from step 0) and the block count
    step = 0
    while step < len(order) and lens[order[step]] == 0:
        step += 1
    any_ = step < len(order)
    kp0 = kad[order[step]] if any_ else 0
    vp0 = vad[order[step]] if any_ else 0
    left0 = lens[order[step]] if any_ else 0
    nb = sum((lens[order[st]] + 31) // 32 for st in range(len(order)))
    return dict(ctp=ctp, end=len(order), nb=nb, kp0=kp0, vp0=vp0, left0=left0, step0=step, kvl=0, kvh=0,
                sbytes=256, blkb=32 * 256, ooff=OOFF, loff=LOFF, koff=KOFF, voff=VOFF)


def _row_addrs(mv, base=0):
    lane = np.arange(64)
    l32, g = lane & 31, lane >> 5
    sw = np.vectorize(swz)
    for ks in range(8):
        mv[ks] = base + l32 * 256 + (((2 * ks + g) ^ sw(l32)) << 4)


def _tr_addrs(mv, first, base):
    lane = np.arange(64)
    g = lane >> 5
    sw = np.vectorize(swz)
    j, sr, m = lane >> 4, (lane >> 2) & 3, lane & 3
    cl = 2 * (j & 1) + (m >> 1)
    for hh in range(2):
        for db in range(4):
            row = 8 * hh + 4 * g + sr
            mv[first + hh * 4 + db] = base + 2 * (row * 128 + (((4 * db + cl) ^ sw(row)) << 3) + 4 * (m & 1))


def _copy_offs(mv, first, w):
    lane = np.arange(64)
    sw = np.vectorize(swz)
    for i in range(2):
        r = (2 * w + i) * 4 + (lane >> 4)
        mv[first + i] = r * 256 + (((lane & 15) ^ sw(r)) << 4)


def _put_rows(regfile, base, rows_bf16, T, w):
    """rows of queries w*64 + 32 qg + l32 (elements 16 ks + 8 g ..) into
    registers base + (8 qg + ks) * 4 (zero past T)"""
    for qg in range(2):
        for ln in range(64):
            qi = w * 64 + qg * 32 + (ln & 31)
            gg = ln >> 5
            for ks in range(8):
                e = (rows_bf16[qi, ks * 16 + gg * 8: ks * 16 + gg * 8 + 8].astype(np.uint32) if qi < T
                     else np.zeros(8, dtype=np.uint32))
                for jj in range(4):
                    regfile[base + (qg * 8 + ks) * 4 + jj, ln] = e[2 * jj] | (e[2 * jj + 1] << 16)


def run_dq_block(q, do, ks, vs, lens, order, stats0, stats1, scale, lines=None):
    """dQ of query rows 0..255 (T = len(q) <= 256) over the chunks; stats
    planes as the dQ kernel computes them (bwd_stat_lse and -D).  Returns dQ
    [T, 128] (scaled)."""
    T = q.shape[0]
    mem = Mem()
    ops0 = _chunk_setup(mem, ks, vs, lens, order)
    c2 = np.float32(scale * 1.4426950408889634)
    lds = np.zeros(LDS_BYTES, dtype=np.uint8)
    waves = []
    for w in range(4):
        wv = Wave(w)
        _put_rows(wv.a, 128, q, T, w)
        _put_rows(wv.a, 192, do, T, w)
        mv = np.zeros((32, 64), dtype=np.int64)
        _row_addrs(mv)
        mv[8:16] = mv[0:8] + 65536
        _tr_addrs(mv, 16, 0)
        _copy_offs(mv, 24, w)
        lane = np.arange(64)
        for qg in range(2):
            qi = w * 64 + qg * 32 + (lane & 31)
            ok = qi < T
            lse2 = np.where(ok, -stats0[np.minimum(qi, T - 1)] * c2, np.inf).astype(np.float32)
            mv[26 + qg] = lse2.view(np.uint32)
            negd = np.where(ok, stats1[np.minimum(qi, T - 1)], 0.0).astype(np.float32).view(np.uint32)
            wv.v[16 * qg:16 * qg + 16] = negd[None, :]
        wv.v[32:64] = mv.astype(np.uint32)
        waves.append(wv)
    ops = [dict(ops0, c2=float(c2), dbase=w * 2048) for w in range(4)]
    lines = [ln.replace('%=', '0') for ln in (lines or GQ.build())]
    _lockstep(lines, ops, mem, lds, waves)
    dq = np.zeros((T, 128))
    for w in range(4):
        af = waves[w].a.view(np.float32)
        for qg in range(2):
            for db in range(4):
                for r in range(16):
                    for ln in range(64):
                        qi = w * 64 + qg * 32 + (ln & 31)
                        if qi < T:
                            d = db * 32 + 8 * (r // 4) + 4 * (ln >> 5) + r % 4
                            dq[qi, d] = af[64 * qg + 16 * db + r, ln] * scale
    return dq


def run_fwd_block(q, ks, vs, lens, order, scale, lines=None):
    """forward of query rows 0..255 over the chunks: O [T, 128], m (natural
    log units: the loop's reference point, within 8 log2 units below the row
    max of the scaled scores; -inf for a row without keys) and l (relative
    to m)."""
    T = q.shape[0]
    mem = Mem()
    ops0 = _chunk_setup(mem, ks, vs, lens, order)
    c2 = np.float32(scale * 1.4426950408889634)
    lds = np.zeros(LDS_BYTES, dtype=np.uint8)
    waves = []
    ninf = np.float32(-np.inf).view(np.uint32)
    for w in range(4):
        wv = Wave(w)
        _put_rows(wv.a, 128, q, T, w)
        mv = np.zeros((32, 64), dtype=np.int64)
        _row_addrs(mv)
        _tr_addrs(mv, 8, 65536)
        _copy_offs(mv, 16, w)
        for i in (18, 19, 26, 27):
            mv[i] = ninf
        wv.v[32:64] = mv.astype(np.uint32)
        m2 = np.zeros((32, 64), dtype=np.uint32)
        m2[1] = 4 * (np.arange(64) >> 5)
        m2[2] = ninf
        wv.v[192:224] = m2
        waves.append(wv)
    ops = [dict(ops0, c2=float(c2), dbase=w * 2048) for w in range(4)]
    lines = [ln.replace('%=', '0') for ln in (lines or GF.build())]
    _lockstep(lines, ops, mem, lds, waves)
    O = np.zeros((T, 128))
    m_out = np.zeros(T)
    l_out = np.zeros(T)
    for w in range(4):
        vf = waves[w].v.view(np.float32)
        af = waves[w].a.view(np.float32)
        for qg in range(2):
            m_ref, l = vf[50 + qg], vf[54 + qg]
            l_tot = l + np.roll(l, 32)
            for ln in range(64):
                qi = w * 64 + qg * 32 + (ln & 31)
                if qi >= T:
                    continue
                inv = 1.0 / l_tot[ln] if l_tot[ln] > 0 else 0.0
                for db in range(4):
                    for r in range(16):
                        d = db * 32 + 8 * (r // 4) + 4 * (ln >> 5) + r % 4
                        O[qi, d] = af[64 * qg + 16 * db + r, ln] * inv
                m_out[qi] = float(m_ref[ln]) * np.log(2.0) if l_tot[ln] > 0 else -np.inf
                l_out[qi] = float(l_tot[ln])
    return O, m_out, l_out


def attention_reference(q, ks, vs, lens, scale):
    """fp64 forward and (with dO) the pieces of the backward over the valid
    keys of every chunk: O, LSE, m (row max of the scaled scores)"""
    Q = bf2f(q.astype(np.uint32)).astype(np.float64)
    K = np.concatenate([bf2f(k[:n].astype(np.uint32)).astype(np.float64) for k, n in zip(ks, lens)])
    V = np.concatenate([bf2f(v[:n].astype(np.uint32)).astype(np.float64) for v, n in zip(vs, lens)])
    S = Q @ K.T * scale
    m = S.max(axis=1)
    P = np.exp(S - m[:, None])
    lsum = P.sum(axis=1)
    P = P / lsum[:, None]
    return P @ V, m + np.log(lsum), m, P, K, V
