"""Generator of the key loop of attn8_kernel (csrc/attention.hip): one inline-asm block per work item, written to
csrc/attn_ring64.inc. Run from the repository root (the build calls it):

    python3 onereel_amd/csrc/gen_attn_ring64.py [--ring 8]

Why asm: a wavefront here owns 64 queries (two 32-query column blocks), so its O accumulators (64 x 128 fp32 =
128 registers per lane) must stay in AGPRs for the whole key loop while S, P and the K/V operands use VGPRs. hipcc
does not keep such a split from source (it moves accumulators between the register files every block), so the loop is
emitted here with fixed registers:

    a0..a127    O^T accumulators, acc(qb, db) = a[64 qb + 16 db : +15]
    a128..a191  Q: k-step k of query block qb at a[128 + 32 qb + 4 k : +3], the MFMAs' B operand
    v36..v99    S, s(par, qb) = v[36 + 32 par + 16 qb : +15] (par = key block parity; S(j+1) fills while S(j) is read)
    v100..v131  P as bf16 pairs, p(par, qb, half) = v[100 + 16 par + 8 qb + 4 half : +3]
    v132..v163  K operands of the 8 k-steps, v164..v195 V^T operands of the 8 (half, db) steps
    v196..v227  -m per query block, broadcast over 16 registers: the first QK^T MFMA of a block accumulates onto it
    v228..v254  softmax temporaries, running max, row sums, LDS read addresses
    s64..s97    K and V buffer descriptors, their remaining byte counts, loop counters, return address, the K and
                V streams' switch points and bases, the prefetched value event and the value event list
The kernel puts Q into a128..a191 before the block (ONEREEL_RING64_QLOAD, or ONEREEL_RING64_QSET_STEP for queries
rotated on the load), or the previous item's block left it there: at its loop's exit, where Q is no longer read, a
block loads the queries of the work-group's next item into those registers (%[qa0], %[qa1]: the lane's query rows of
that item, or of this item when the next one is not claimed yet: the 16 loads are unconditional), so that these loads
are not queued behind its O stores in the in-order vmcnt.
S = q k^T - m comes out of the MFMAs (the first of each block accumulates onto -m), so P = 2^(c S), c = scale *
log2(e), takes one v_mul_f32 and one v_exp_f32 per score: the fp32 scores of FlashAttention's exp2(s c - m c), with
the subtraction folded into the accumulator.

Schedule of iteration j (32 keys; R-slot rings of K and V blocks in LDS, 8 KiB per slot):
    phase A  MFMA steps k = 0..3: S(j+1) += K(j+1)_k Q_k^T for both query blocks, O += V(j-1)_k P(j-1)_k; the VALU
             computes P(j) of query block 0 in between; the LDS operands of steps 4..7 are read
    mid      wait until this wavefront's loads of K(j+2), V(j) have landed, barrier; DMA of K(j+R) into slot j % R and
             of V(j+R-2) into slot (j-2) % R (both consumed by iteration j-1) goes out during phase B
    phase B  steps k = 4..7, P(j) of query block 1, and the LDS operands of steps 0..3 of iteration j+1
    tail     if the lane's two row-half sums of P(j) (one per query block) add up to more than 2^20 (or are not
             finite): out-of-line rescale (per query block, m moves up by d = max(block max, 0), O and l scale by
             2^(-c d), S(j), S(j+1) and -m shift by -d, P(j) recomputed). One compare of the sum instead of one
             per query block leaves the scalar branch a single VALU result to wait for, and the loop's end test
             fills that wait; then l += row sums
    end      one scalar branch, taken at j + 1 >= nb - 1: out of line, either the loop's exit or the mask of the last
             block's scores (keys past the segment -> -inf) before the last iteration. Each branch of an iteration
             costs the MFMA pipe: a separate mask check at the iteration's start made the kernel 1.3% slower
Within a phase the eight S MFMAs go before the eight PV MFMAs, and the side work (softmax VALU, LDS reads, DMA) is
spread between them in proportion to its issue cost (SIDE_COST).
The running max starts at block 0's own maximum (prologue), so row sums never underflow and m only moves up.
After the loop: the next item's Q loads, the epilogue (O += V(nb-1) P(nb-1)) and the store of O / l, as bf16 output
rows or, for the parts of a key-split work item, as fp32 partial rows (%[f32]). A wavefront whose queries all lie
past the segment (%[dead]) runs a loop of only the barriers and its share of the DMA, so that the block stays in
step, issues the next item's Q loads at its exit and writes nothing; it leaves the block before the others'
epilogues, so the kernel waits for a barrier before it refills the ring for the next item.
In-place keys and values: V blocks 0 .. nbav-1 (%[nbav]) are read from token-order value rows (the descriptor's first
base, %[vb_lo] / %[vb_hi]), the others from the packed rows (%[vsw]: the base of block nbav there; both advance by
%[bb] per block), and K blocks 0 .. nbak-1 likewise (%[ksw]). Each base is replaced with no cost in the steady-state
loop: in the ring fill (V: nbav <= R - 2; K: nbak <= R, the kernel's ring head covering nbak <= 2), else at the end of
the iteration whose refill fetched the block before the switch, which the loop's end test already stops at (its
bound is the least of nb - 1 and those iterations). The value stream may move more than once (value runs: shared
frames read in place between packed rows): each move takes the next event from the item's event list (%[vlist]:
16-byte entries of block, base lo, base hi, for head 0; %[hoff] adds the head's offset, %[b0] makes the block
relative to the item's first), whose entry after the next is prefetched with a scalar load one event ahead.
The generator inserts the LDS waits (lgkmcnt) from the order of the reads, and s_nop where gfx950 needs wait states
between dependent instructions (see Emitter).
"""
from __future__ import annotations

import argparse
from pathlib import Path

SLOT = 8192              # bytes per K or V block: 32 keys x 128 dims x bf16
MFMA_WAIT = 12           # wait states between a 32x32x16 bf16 MFMA and a VALU / memory access to its result
LGKM_MAX = 15


# fixed registers
def S(par, qb, r):
    return 36 + 32 * par + 16 * qb + r


def Sx(par, qb):
    b = S(par, qb, 0)
    return f'v[{b}:{b + 15}]'


def P(par, qb, half, i):
    return 100 + 16 * par + 8 * qb + 4 * half + i


def Px(par, qb, half):
    b = P(par, qb, half, 0)
    return f'v[{b}:{b + 3}]'


def KOP(k):
    return 132 + 4 * k


def VOP(k):
    return 164 + 4 * k


def MCV(qb):
    return 196 + 16 * qb


T0, A0, TT, LS0, M0, LSUM0, KADDR0, VADDR0 = 228, 232, 236, 237, 239, 241, 243, 251
FIRST_FIXED = 36


def QA(qb, k):
    return 128 + 32 * qb + 4 * k


def ACC(qb, db):
    b = 64 * qb + 16 * db
    return f'a[{b}:{b + 15}]'


KRES, VRES = 64, 68             # s[64:67], s[68:71]
KREM, VREM, SJ, SNB1, SRR, SVOFF = 72, 73, 74, 75, 76, 77
SRA, SX, SEX = 78, 80, 82       # s[78:79], s[80:81], s[82:83]
SVTHR, SVSW = 84, 86            # s84: loop count at which the V stream leaves the in-place rows; s[86:87]: its new base
SKTHR, SKSW, STMP = 85, 88, 90  # s85, s[88:89]: the same for the K stream; s90: a temporary of the end test
SLD, SVL = 92, 96               # s[92:95]: the value event after the next one (prefetched); s[96:97]: the list's next entry
LAST_SGPR = 97
NEG_INF = '0xff800000'


def v(x):
    return f'v{x}'


class Emitter:
    """Straight-line code with two trackers: outstanding LDS reads (for lgkmcnt) and the registers recent VALU,
    transcendental and MFMA instructions wrote (for the wait states gfx950 needs before they are read; hipcc inserts
    the same s_nop counts for these patterns):
        MFMA result          -> VALU / memory access   12 wait states
        v_exp / v_rcp result -> VALU read               1
        VALU result          -> MFMA source             2
        VALU result          -> v_permlane32_swap       2"""

    def __init__(self):
        self.lines = []
        self.pos = 0              # position of the next instruction, in wait states
        self.lds = []             # outstanding LDS reads: list of sets of destination VGPRs, in issue order
        self.mfma_w = {}          # register -> position of the MFMA that wrote it
        self.trans_w = {}         # register -> position of the transcendental that wrote it
        self.valu_w = {}          # register -> position of the VALU instruction that wrote it

    def raw(self, s, cost=1):
        self.lines.append(s)
        self.pos += cost

    def label(self, name):
        self.lines.append(f'{name}:')

    def nop_to(self, need):
        while need > 0:
            n = min(need, 8)
            self.raw(f's_nop {n - 1}', n)
            need -= n

    def _regs(self, regs):
        out = set()
        for r in regs:
            if isinstance(r, tuple):
                kind, lo, n = r
                out.update(f'{kind}{lo + i}' for i in range(n))
            else:
                out.add(r)
        return out

    def wait_lds(self, regs):
        regs = self._regs(regs)
        last = -1
        for i, dst in enumerate(self.lds):
            if dst & regs:
                last = i
        if last >= 0:
            after = len(self.lds) - last - 1
            self.raw(f's_waitcnt lgkmcnt({min(after, LGKM_MAX)})')
            del self.lds[:last + 1]

    def wait_lds_all(self):
        if self.lds:
            self.raw('s_waitcnt lgkmcnt(0)')
            self.lds = []

    def _need(self, table, regs, waits):
        need = 0
        for r in regs:
            p = table.get(r)
            if p is not None:
                need = max(need, p + 1 + waits - self.pos)
        return need

    def valu(self, s, reads=(), writes=(), trans=False, permlane=False):
        rd, wr = self._regs(reads), self._regs(writes)
        self.wait_lds(list(rd | wr))
        need = max(self._need(self.mfma_w, rd | wr, MFMA_WAIT), self._need(self.trans_w, rd, 1),
                   self._need(self.valu_w, rd, 2) if permlane else 0)
        self.nop_to(need)
        at = self.pos
        self.raw(s)
        for r in wr:
            self.valu_w[r] = at
            if trans:
                self.trans_w[r] = at
            else:
                self.trans_w.pop(r, None)
            self.mfma_w.pop(r, None)

    def ds_read(self, s, dst):
        d = self._regs(dst)
        self.nop_to(self._need(self.mfma_w, d, MFMA_WAIT))
        self.lds.append(d)
        self.raw(s)

    def mfma(self, dst, a, b, c, dst_regs, read_regs):
        self.wait_lds(read_regs)
        self.nop_to(self._need(self.valu_w, self._regs(read_regs), 2))
        at = self.pos
        self.raw(f'v_mfma_f32_32x32x16_bf16 {dst}, {a}, {b}, {c}')
        for r in self._regs(dst_regs):
            self.mfma_w[r] = at


def vr(lo, n=1):
    return ('v', lo, n)


# relative cost of a side op ('valu', asm, reads, writes, trans) or ('m0' | 'dma' | 'raw', asm) when spreading the
# side ops of a phase between its 16 MFMAs. A transcendental takes the VALU four times as long as an fp32 op, and an
# LDS DMA issue holds the wavefront longer than an ALU op; these weights were the fastest of a sweep (trans 1.5-4,
# dma 1-4, MFMA order): 2.7-3% faster than equal weights with S and PV MFMAs alternating by k-step.
SIDE_COST = {'valu': 1.0, 'trans': 2.0, 'm0': 1.0, 'dma': 3.0, 'raw': 1.0}


def side_cost(op):
    if op[0] == 'valu':
        return SIDE_COST['trans' if op[4] else 'valu']
    return SIDE_COST[op[0]]


def v_advance(R):
    """the value stream moves to the next event's base (s[86:87]); the prefetched event (s[92:95]: block, base lo,
    base hi) becomes the next one (its loop count in s84: block - b0 - (R - 2), or never past the item), and the
    event after it is prefetched. The prefetch was issued an event earlier (or in the prologue), so the wait finds it
    landed; a wait for all LDS reads too costs little at an iteration's end."""
    return [f's_mov_b64 s[{VRES}:{VRES + 1}], s[{SVSW}:{SVSW + 1}]',
            's_waitcnt lgkmcnt(0)',
            f's_add_u32 s{SVSW}, s{SLD + 1}, %[hoff]',
            f's_addc_u32 s{SVSW + 1}, s{SLD + 2}, 0',
            f's_sub_u32 s{STMP}, s{SLD}, %[b0]',
            f's_cmp_lt_u32 s{STMP}, %[nb]',
            f's_cselect_b32 s{STMP}, s{STMP}, 0x7fffffff',
            f's_sub_u32 s{SVTHR}, s{STMP}, {R - 2}',
            f's_cmp_eq_u32 s{STMP}, 0x7fffffff',
            f's_cselect_b32 s{SVTHR}, 0x7fffffff, s{SVTHR}',
            f's_load_dwordx4 s[{SLD}:{SLD + 3}], s[{SVL}:{SVL + 1}], 0x0',
            f's_add_u32 s{SVL}, s{SVL}, 16',
            f's_addc_u32 s{SVL + 1}, s{SVL + 1}, 0']


class Kernel:
    def __init__(self, ring):
        assert ring in (4, 6, 8)
        self.R = ring
        self.VBASE = ring * SLOT      # V ring after the K ring

    # ---- pieces ------------------------------------------------------------------------------------------------
    def dma(self, e, res, rem, vo, lds_off):
        for n in range(2):
            e.raw(f's_add_u32 m0, %[sbase], {lds_off + n * 4096}')
            e.raw('s_nop 0')                      # gfx9: an SALU write of M0 and the LDS DMA reading it
            e.raw(f'buffer_load_dwordx4 %[{vo}{n}], s[{res}:{res + 3}], 0 offen lds')
        e.raw(f's_add_u32 s{res}, s{res}, %[bb]')
        e.raw(f's_addc_u32 s{res + 1}, s{res + 1}, 0')
        e.raw(f's_sub_i32 s{rem}, s{rem}, %[bb]')
        e.raw(f's_max_i32 s{res + 2}, s{rem}, 0')

    def dma_k(self, e, slot):
        self.dma(e, KRES, KREM, 'vk', slot * SLOT)

    def dma_v(self, e, slot):
        self.dma(e, VRES, VREM, 'vv', self.VBASE + slot * SLOT)

    def dma_ops(self, J):
        """the mid-iteration refill as side ops: K(j+R) into slot J, V(j+R-2) into slot (J-2) % R"""
        R = self.R
        ops = []
        for res, rem, slot_off, vo in ((KRES, KREM, (J % R) * SLOT, 'vk'),
                                       (VRES, VREM, self.VBASE + ((J - 2) % R) * SLOT, 'vv')):
            for n in range(2):
                ops.append(('m0', f's_add_u32 m0, %[sbase], {slot_off + n * 4096}'))
                ops.append(('dma', f'buffer_load_dwordx4 %[{vo}{n}], s[{res}:{res + 3}], 0 offen lds'))
            ops.append(('raw', f's_add_u32 s{res}, s{res}, %[bb]'))
            ops.append(('raw', f's_addc_u32 s{res + 1}, s{res + 1}, 0'))
            ops.append(('raw', f's_sub_i32 s{rem}, s{rem}, %[bb]'))
            ops.append(('raw', f's_max_i32 s{res + 2}, s{rem}, 0'))
        return ops

    def read_k(self, e, k, slot):
        e.ds_read(f'ds_read_b128 v[{KOP(k)}:{KOP(k) + 3}], v{KADDR0 + k} offset:{slot * SLOT}', [vr(KOP(k), 4)])

    def read_v(self, e, k, slot, addr=None):
        half, db = divmod(k, 4)
        a = addr if addr is not None else f'v{VADDR0 + db}'
        for t in range(2):
            lo = VOP(k) + 2 * t
            e.ds_read(f'ds_read_b64_tr_b16 v[{lo}:{lo + 1}], {a} offset:{slot * SLOT + (8 * half + 4 * t) * 256}',
                      [vr(lo, 2)])

    def softmax(self, par, qb):
        """P(par, qb) = bf16(2^(c S)) and LS(qb) = fp32 sum of the unrounded values: list of (asm, reads, writes,
        trans)"""
        T = lambda r: T0 + (r % 4)

        def mul(p):
            return [(f'v_mul_f32_e32 v{T(r)}, %[c], v{S(par, qb, r)}', [v(S(par, qb, r))], [v(T(r))], False)
                    for r in (2 * p, 2 * p + 1)]

        def exp(p):
            return [(f'v_exp_f32_e32 v{T(r)}, v{T(r)}', [v(T(r))], [v(T(r))], True) for r in (2 * p, 2 * p + 1)]

        def tail(p):
            r0, r1 = 2 * p, 2 * p + 1
            half, i = divmod(p, 4)
            out = [(f'v_cvt_pk_bf16_f32 v{P(par, qb, half, i)}, v{T(r0)}, v{T(r1)}', [v(T(r0)), v(T(r1))],
                    [v(P(par, qb, half, i))], False)]
            if p < 4:
                out.append((f'v_add_f32_e32 v{A0 + p}, v{T(r0)}, v{T(r1)}', [v(T(r0)), v(T(r1))], [v(A0 + p)], False))
            else:
                out.append((f'v_add_f32_e32 v{TT}, v{T(r0)}, v{T(r1)}', [v(T(r0)), v(T(r1))], [v(TT)], False))
                out.append((f'v_add_f32_e32 v{A0 + p - 4}, v{A0 + p - 4}, v{TT}', [v(A0 + p - 4), v(TT)],
                            [v(A0 + p - 4)], False))
            return out

        # pair p: c*S, 2^(c*S) one pair ahead of its cvt and adds (no transcendental result is read by the next
        # instruction); a pair's T registers are rewritten only after its tail has read them
        ops = mul(0)
        for p in range(8):
            ops += exp(p)
            if p >= 1:
                ops += tail(p - 1)
            if p + 1 < 8:
                ops += mul(p + 1)
        ops.append((f'v_add_f32_e32 v{A0}, v{A0}, v{A0 + 1}', [v(A0), v(A0 + 1)], [v(A0)], False))
        ops += tail(7)
        ops.append((f'v_add_f32_e32 v{A0 + 2}, v{A0 + 2}, v{A0 + 3}', [v(A0 + 2), v(A0 + 3)], [v(A0 + 2)], False))
        ops.append((f'v_add_f32_e32 v{LS0 + qb}, v{A0}, v{A0 + 2}', [v(A0), v(A0 + 2)], [v(LS0 + qb)], False))
        return ops

    def mfma_s(self, e, par_next, qb, k, seed=None):
        """S(par_next, qb) += K_k Q_k^T; the first step accumulates onto -m (or onto `seed`)"""
        if k == 0:
            c = seed if seed is not None else f'v[{MCV(qb)}:{MCV(qb) + 15}]'
            reads = [vr(KOP(k), 4)] + ([] if seed is not None else [vr(MCV(qb), 16)])
        else:
            c = Sx(par_next, qb)
            reads = [vr(KOP(k), 4), vr(S(par_next, qb, 0), 16)]
        e.mfma(Sx(par_next, qb), f'v[{KOP(k)}:{KOP(k) + 3}]', f'a[{QA(qb, k)}:{QA(qb, k) + 3}]', c,
               [vr(S(par_next, qb, 0), 16)], reads)

    def mfma_pv(self, e, par_prev, qb, k):
        half, db = divmod(k, 4)
        e.mfma(ACC(qb, db), f'v[{VOP(k)}:{VOP(k) + 3}]', Px(par_prev, qb, half), ACC(qb, db), [],
               [vr(VOP(k), 4), vr(P(par_prev, qb, half, 0), 4)])

    def row_max(self, e, par, qb, dst, tmp):
        """dst = max over the query's 32 scores of block par (in-lane 16, then with lane ^ 32)"""
        s = [S(par, qb, r) for r in range(16)]
        e.valu(f'v_max3_f32 v{dst}, v{s[0]}, v{s[1]}, v{s[2]}', [v(s[0]), v(s[1]), v(s[2])], [v(dst)])
        for r in range(3, 15, 2):
            e.valu(f'v_max3_f32 v{dst}, v{dst}, v{s[r]}, v{s[r + 1]}', [v(dst), v(s[r]), v(s[r + 1])], [v(dst)])
        e.valu(f'v_max_f32_e32 v{dst}, v{dst}, v{s[15]}', [v(dst), v(s[15])], [v(dst)])
        e.valu(f'v_mov_b32_e32 v{tmp}, v{dst}', [v(dst)], [v(tmp)])
        e.valu(f'v_permlane32_swap_b32_e32 v{dst}, v{tmp}', [v(dst), v(tmp)], [v(dst), v(tmp)], permlane=True)
        e.valu(f'v_max_f32_e32 v{dst}, v{dst}, v{tmp}', [v(dst), v(tmp)], [v(dst)])

    def mask(self, e, par):
        """scores of keys past the segment's end -> -inf (S(j) of the segment's last block)"""
        e.valu(f'v_mov_b32_e32 v{T0}, {NEG_INF}', [], [v(T0)])
        for r in range(16):
            e.valu(f'v_cmp_lt_i32_e32 vcc, {r}, %[valid]', [], [])
            for qb in range(2):
                e.valu(f'v_cndmask_b32_e32 v{S(par, qb, r)}, v{T0}, v{S(par, qb, r)}, vcc',
                       [v(T0), v(S(par, qb, r))], [v(S(par, qb, r))])

    # ---- one iteration -------------------------------------------------------------------------------------------
    def body(self, e, J):
        """one iteration: 32 MFMAs with the softmax, LDS reads and DMA spread between them. Every LDS operand is
        read half an iteration ahead, so each phase starts with one lgkmcnt(0) and its MFMAs wait for nothing else."""
        R = self.R
        par, npar = J & 1, (J & 1) ^ 1
        e.label(f'.Lmaskret{J}_%=')
        ks_now, vs_now = (J + 1) % R, (J - 1) % R          # slots of K(j+1), V(j-1)
        ks_next, vs_next = (J + 2) % R, J % R               # slots of K(j+2), V(j)

        def reads(kslot, vslot, ks):
            out = []
            for k in ks:
                out.append(('k', k, kslot))
                out.append(('v', k, vslot))
            return out

        def emit_side(op, last_m0):
            if op[0] == 'valu':
                e.valu(op[1], op[2], op[3], trans=op[4])
            elif op[0] == 'dma' and last_m0:
                e.nop_to(1)
                e.raw(op[1])
            else:
                e.raw(op[1])
            return op[0] == 'm0'

        def phase(ks, valu_ops, rd, dma):
            e.wait_lds_all()
            side = [('valu',) + op for op in valu_ops]
            if dma:
                # one VALU op between each M0 write and its load (gfx9 LDS-DMA M0 hazard)
                merged, vi = [], 0
                for op in dma:
                    merged.append(op)
                    if op[0] == 'm0' and vi < len(side):
                        merged.append(side[vi])
                        vi += 1
                side = merged + side[vi:]
            # the eight S MFMAs of the phase (both column blocks, k-steps interleaved), then the eight PV MFMAs: S(j+1)
            # is complete eight MFMAs before the next iteration's softmax reads it
            order = ([('s', qb, k) for k in ks for qb in (0, 1)] +
                     [('pv', qb, k) for k in ks for qb in (0, 1)])
            # side ops go between the MFMAs in proportion to their issue cost (SIDE_COST)
            cost = [side_cost(op) for op in side]
            total = float(sum(cost))
            done, spent, last_m0 = 0, 0.0, False
            for i, (kind, qb, k) in enumerate(order):
                if kind == 's':
                    self.mfma_s(e, npar, qb, k)
                else:
                    self.mfma_pv(e, npar, qb, k)
                if rd:
                    kr_kind, kr, slot = rd.pop(0)
                    (self.read_k if kr_kind == 'k' else self.read_v)(e, kr, slot)
                target = total * (i + 1) / 16.0
                while done < len(side) and spent + 0.5 * cost[done] < target:
                    last_m0 = emit_side(side[done], last_m0)
                    spent += cost[done]
                    done += 1
            while done < len(side):
                last_m0 = emit_side(side[done], last_m0)
                done += 1

        phase([0, 1, 2, 3], self.softmax(par, 0), reads(ks_now, vs_now, range(4, 8)), None)
        # mid: K(j+2), V(j) landed (this wavefront's loads) and visible (barrier); the refill of the freed slots goes
        # out during phase B
        e.raw(f's_waitcnt vmcnt({4 * (R - 3)})')
        e.raw('s_barrier')
        phase([4, 5, 6, 7], self.softmax(par, 1), reads(ks_next, vs_next, range(4)), self.dma_ops(J))
        # rescale check on the sum of the lane's two row-half sums (a sum over 2^20, or not finite, rescales both
        # query blocks; one with no new maximum keeps its m), then the row sums
        e.valu(f'v_add_f32_e32 v{TT}, v{LS0}, v{LS0 + 1}', [v(LS0), v(LS0 + 1)], [v(TT)])
        e.valu(f'v_cmp_nge_f32_e32 vcc, s{SRR}, v{TT}', [v(TT)])
        # the loop's end test fills the wait for the compare (the rescale block sets SCC again before it returns)
        e.raw(f's_add_u32 s{SJ}, s{SJ}, 1')
        e.raw(f's_cmp_ge_u32 s{SJ}, s{SNB1}')
        e.raw(f's_getpc_b64 s[{SRA}:{SRA + 1}]')
        e.raw(f's_cbranch_vccnz .Lrescale{par}_%=')
        e.valu(f'v_add_f32_e32 v{LSUM0}, v{LSUM0}, v{LS0}', [v(LSUM0), v(LS0)], [v(LSUM0)])
        e.valu(f'v_add_f32_e32 v{LSUM0 + 1}, v{LSUM0 + 1}, v{LS0 + 1}', [v(LSUM0 + 1), v(LS0 + 1)], [v(LSUM0 + 1)])
        # one branch per iteration for the loop's end and the last block's mask: at j + 1 >= nb - 1 the out-of-line
        # code either leaves the loop or masks S(nb - 1) before the last iteration
        e.raw(f's_cbranch_scc1 .Lend{J}_%=')

    def end_block(self, J):
        """after iteration J with j + 1 >= s75 = min(nb - 1, s84, s85): at j + 1 = s84 the V stream's base moves to
        the packed rows (%[vsw]: the next refill fetches block nbav), at j + 1 = s85 the K stream's (%[ksw], block
        nbak); s75 becomes the least of nb - 1 and the switch points still ahead. Then, below nb - 1, go on with the
        next iteration; at j + 1 >= nb - 1 leave the loop when j + 1 = nb, else mask the last block first"""
        R = self.R
        return [f'.Lend{J}_%=:',
                f's_cmp_eq_u32 s{SJ}, s{SVTHR}',
                f's_cbranch_scc0 .Lvn{J}_%='] + v_advance(R) + [
                f'.Lvn{J}_%=:',
                f's_cmp_eq_u32 s{SJ}, s{SKTHR}',
                f's_cselect_b64 s[{KRES}:{KRES + 1}], s[{SKSW}:{SKSW + 1}], s[{KRES}:{KRES + 1}]',
                f's_sub_u32 s{SNB1}, %[nb], 1',
                f's_cmp_gt_u32 s{SVTHR}, s{SJ}', f's_cselect_b32 s{STMP}, s{SVTHR}, s{SNB1}',
                f's_min_u32 s{SNB1}, s{SNB1}, s{STMP}',
                f's_cmp_gt_u32 s{SKTHR}, s{SJ}', f's_cselect_b32 s{STMP}, s{SKTHR}, s{SNB1}',
                f's_min_u32 s{SNB1}, s{SNB1}, s{STMP}',
                f's_cmp_lt_u32 s{SJ}, s{SNB1}', f's_cbranch_scc1 .Lmaskret{(J + 1) % R}_%=',
                f's_cmp_ge_u32 s{SJ}, %[nb]', f's_cbranch_scc1 .Lexit{J}_%=',
                f's_branch .Lmask{(J + 1) % R}_%=']

    def mask_block(self, J):
        e = Emitter()
        e.label(f'.Lmask{J}_%=')
        e.nop_to(MFMA_WAIT)
        self.mask(e, J & 1)
        e.raw(f's_branch .Lmaskret{J}_%=')
        return e.lines

    def rescale_block(self, par):
        """entered after the MFMAs of the iteration (20 wait states before S or the accumulators are touched): the
        running max moves up by d = max(block max, 0) >= 0; O and l scale by 2^(-c d); S(j), S(j+1) (accumulated onto
        the old -m) and -m shift by -d; P(j) and its row sums are recomputed"""
        npar = par ^ 1
        e = Emitter()
        e.label(f'.Lrescale{par}_%=')
        e.nop_to(20)
        d, alpha = A0, A0 + 1            # free until the softmax recompute
        for qb in range(2):
            self.row_max(e, par, qb, d, alpha)
            e.valu(f'v_max_f32_e32 v{d}, 0, v{d}', [v(d)], [v(d)])
            e.valu(f'v_mul_f32_e32 v{alpha}, %[c], v{d}', [v(d)], [v(alpha)])
            e.valu(f'v_exp_f32_e64 v{alpha}, -v{alpha}', [v(alpha)], [v(alpha)], trans=True)
            e.valu(f'v_add_f32_e32 v{M0 + qb}, v{M0 + qb}, v{d}', [v(M0 + qb), v(d)], [v(M0 + qb)])
            for r in range(16):
                for reg in (S(par, qb, r), S(npar, qb, r), MCV(qb) + r):
                    e.valu(f'v_sub_f32_e32 v{reg}, v{reg}, v{d}', [v(reg), v(d)], [v(reg)])
            e.valu(f'v_mul_f32_e32 v{LSUM0 + qb}, v{LSUM0 + qb}, v{alpha}', [v(LSUM0 + qb), v(alpha)],
                   [v(LSUM0 + qb)])
            for base in range(0, 64, 4):
                acc = [64 * qb + base + i for i in range(4)]
                for i in range(4):
                    e.valu(f'v_accvgpr_read_b32 v{T0 + i}, a{acc[i]}', [], [v(T0 + i)])
                for i in range(4):
                    e.valu(f'v_mul_f32_e32 v{T0 + i}, v{T0 + i}, v{alpha}', [v(T0 + i), v(alpha)], [v(T0 + i)])
                for i in range(4):
                    e.valu(f'v_accvgpr_write_b32 a{acc[i]}, v{T0 + i}', [v(T0 + i)], [f'a{acc[i]}'])
            for op, rd, wr, tr in self.softmax(par, qb):
                e.valu(op, rd, wr, trans=tr)
        e.nop_to(2)
        e.raw(f's_add_u32 s{SRA}, s{SRA}, 4')
        e.raw(f's_addc_u32 s{SRA + 1}, s{SRA + 1}, 0')
        e.raw(f's_cmp_ge_u32 s{SJ}, s{SNB1}')        # the iteration's end test, for the branch after the return
        e.raw(f's_setpc_b64 s[{SRA}:{SRA + 1}]')
        return e.lines

    @staticmethod
    def q_prefetch():
        """the next item's queries into a128..a191: issued at the loop's exit, where Q is no longer read and before
        the O stores, which are then the last 16 ... 48 vector memory operations of the block"""
        return [f'global_load_dwordx4 a[{QA(qb, k)}:{QA(qb, k) + 3}], %[qa{qb}], off offset:{32 * k}'
                for qb in range(2) for k in range(8)]

    def epilogue(self, par):
        """the next item's Q loads, then O += V(nb-1) P(nb-1): steps 0..3 were prefetched by the last iteration,
        steps 4..7 are read from the slot whose byte offset is in s77"""
        e = Emitter()
        e.lds = self._regs_prefetch()
        e.label(f'.Lepi{par}_%=')
        for line in self.q_prefetch():
            e.raw(line)
        for db in range(4):
            e.raw(f'v_add_u32_e32 v{T0 + db}, s{SVOFF}, v{VADDR0 + db}')
        for k in range(4, 8):
            self.read_v(e, k, 0, addr=f'v{T0 + k - 4}')
        for k in range(8):
            for qb in range(2):
                self.mfma_pv(e, par, qb, k)
        e.raw(f's_branch .Lstore_%=')
        return e.lines

    def _regs_prefetch(self):
        regs = []
        for k in range(4):
            regs.append({f'v{KOP(k) + i}' for i in range(4)})
            for t in range(2):
                regs.append({f'v{VOP(k) + 2 * t + i}' for i in range(2)})
        return regs

    def store_block(self):
        """O / l to the output rows (rows past the segment masked off): bf16, or fp32 when %[f32] is non-zero (the
        partial results of a work item split by keys); 16 wait states after the last MFMA. The ring's last loads
        have landed before the stores (the next item's 16 Q loads, issued after them, may still be in flight).
        Temporaries live in the S registers, which are dead here."""
        e = Emitter()
        e.label('.Lstore_%=')
        e.nop_to(16)
        e.raw('s_waitcnt vmcnt(16) lgkmcnt(0)')
        x = [S(0, 0, i) for i in (0, 1, 2, 4, 5, 6, 7)]   # v[40:41] is the even-aligned store pair
        for qb in range(2):
            e.valu(f'v_mov_b32_e32 v{x[0]}, v{LSUM0 + qb}', [v(LSUM0 + qb)], [v(x[0])])
            e.valu(f'v_mov_b32_e32 v{x[1]}, v{LSUM0 + qb}', [v(LSUM0 + qb)], [v(x[1])])
            e.valu(f'v_permlane32_swap_b32_e32 v{x[0]}, v{x[1]}', [v(x[0]), v(x[1])], [v(x[0]), v(x[1])],
                   permlane=True)
            e.valu(f'v_add_f32_e32 v{x[0]}, v{x[0]}, v{x[1]}', [v(x[0]), v(x[1])], [v(x[0])])   # l of the query
            e.valu(f'v_mov_b32_e32 %[lo{qb}], v{x[0]}', [v(x[0])], [])
            e.valu(f'v_mov_b32_e32 %[mo{qb}], v{M0 + qb}', [v(M0 + qb)], [])
            e.valu(f'v_rcp_f32_e32 v{x[2]}, v{x[0]}', [v(x[0])], [v(x[2])], trans=True)
            e.valu(f'v_cmp_ne_u32_e32 vcc, 0, %[ok{qb}]', [], [])
            e.raw(f's_and_saveexec_b64 s[{SEX}:{SEX + 1}], vcc')
            e.raw('s_cmp_eq_u32 %[f32], 0')
            e.raw(f's_cbranch_scc0 .Lst32_{qb}_%=')
            for f32 in (False, True):
                if f32:
                    e.raw(f's_branch .Lstdone_{qb}_%=')
                    e.label(f'.Lst32_{qb}_%=')
                for db in range(4):
                    for g in range(4):
                        acc = 64 * qb + 16 * db + 4 * g
                        for i in range(4):
                            e.valu(f'v_accvgpr_read_b32 v{x[3 + i]}, a{acc + i}', [], [v(x[3 + i])])
                        for i in range(4):
                            e.valu(f'v_mul_f32_e32 v{x[3 + i]}, v{x[3 + i]}, v{x[2]}', [v(x[3 + i]), v(x[2])],
                                   [v(x[3 + i])])
                        if f32:
                            # lane half h: dims 32 db + 8 g + 4 h .. + 3 of its query, 16 bytes. A store of more
                            # than 8 bytes reads its data registers after issue: one wait state before they are
                            # rewritten (gfx9 VMEM store-data hazard)
                            e.raw(f'global_store_dwordx4 %[op{qb}], v[{x[3]}:{x[6]}], off offset:{db * 128 + 32 * g}')
                            e.raw('s_nop 0')
                        else:
                            e.valu(f'v_cvt_pk_bf16_f32 v{x[3]}, v{x[3]}, v{x[4]}', [v(x[3]), v(x[4])], [v(x[3])])
                            e.valu(f'v_cvt_pk_bf16_f32 v{x[4]}, v{x[5]}, v{x[6]}', [v(x[5]), v(x[6])], [v(x[4])])
                            e.raw(f'global_store_dwordx2 %[op{qb}], v[{x[3]}:{x[4]}], off offset:{db * 64 + 16 * g}')
            e.label(f'.Lstdone_{qb}_%=')
            e.raw(f's_mov_b64 exec, s[{SEX}:{SEX + 1}]')
        return e.lines

    def prologue(self, e):
        R = self.R
        e.raw('s_waitcnt vmcnt(0) lgkmcnt(0)')
        e.raw(f's_mov_b32 s{SRR}, 0x49800000')      # 2^20
        e.raw(f's_mov_b32 s{SJ}, 0')
        # the value stream moves to %[vsw] at block nbav (0: never) and then at each event of %[vlist]. s84 holds
        # nbav - (R - 2): the ring fill below moves it after its fetch of block nbav - 1 when nbav <= R - 2, else the
        # loop's end test stops at the end of the iteration whose V refill fetched block nbav - 1 (j + 1 = s84);
        # each move takes the next event (v_advance). The event after the next one is prefetched here.
        e.raw(f's_mov_b64 s[{SVSW}:{SVSW + 1}], %[vsw]')
        e.raw(f's_sub_u32 s{SVTHR}, %[nbav], {R - 2}')
        e.raw('s_cmp_eq_u32 %[nbav], 0')
        e.raw(f's_cselect_b32 s{SVTHR}, 0x7fffffff, s{SVTHR}')
        e.raw(f's_mov_b64 s[{SVL}:{SVL + 1}], %[vlist]')
        e.raw(f's_load_dwordx4 s[{SLD}:{SLD + 3}], s[{SVL}:{SVL + 1}], 0x0')
        e.raw(f's_add_u32 s{SVL}, s{SVL}, 16')
        e.raw(f's_addc_u32 s{SVL + 1}, s{SVL + 1}, 0')
        # K blocks 0 .. nbak-1 likewise (%[ksw]: the packed rows of block nbak): the kernel's ring head covers
        # nbak <= 2, the ring fill nbak <= R, the loop's end test the rest (j + 1 = nbak - R, in s85)
        e.raw(f's_mov_b64 s[{SKSW}:{SKSW + 1}], %[ksw]')
        e.raw(f's_add_u32 s{SKTHR}, %[nbak], {-R}')
        e.raw(f's_cmp_lt_u32 %[nbak], {R + 1}')
        e.raw(f's_cselect_b32 s{SKTHR}, 0x7fffffff, s{SKTHR}')
        # the K descriptor starts at block 2 (%[kb_lo], %[kb_hi], %[remk]): the kernel fetched the ring's head
        for res, rem, lo, hi, r0 in ((KRES, KREM, 'kb_lo', 'kb_hi', 'remk'), (VRES, VREM, 'vb_lo', 'vb_hi', 'rem0')):
            e.raw(f's_mov_b32 s{res}, %[{lo}]')
            e.raw(f's_mov_b32 s{res + 1}, %[{hi}]')
            e.raw(f's_mov_b32 s{rem}, %[{r0}]')
            e.raw(f's_max_i32 s{res + 2}, s{rem}, 0')
            e.raw(f's_mov_b32 s{res + 3}, 0x20000')
        e.valu(f'v_mov_b32_e32 v{KADDR0}, %[kb]', [], [v(KADDR0)])
        for k in range(1, 8):
            e.valu(f'v_xor_b32_e32 v{KADDR0 + k}, {32 * k}, %[kb]', [], [v(KADDR0 + k)])
        e.valu(f'v_mov_b32_e32 v{VADDR0}, %[vb]', [], [v(VADDR0)])
        for db in range(1, 4):
            e.valu(f'v_xor_b32_e32 v{VADDR0 + db}, {64 * db}, %[vb]', [], [v(VADDR0 + db)])
        for qb in range(2):
            e.valu(f'v_mov_b32_e32 v{LSUM0 + qb}, 0', [], [v(LSUM0 + qb)])
            for half in range(2):
                for i in range(4):
                    e.valu(f'v_mov_b32_e32 v{P(1, qb, half, i)}, 0', [], [v(P(1, qb, half, i))])
        for i in range(128):
            e.valu(f'v_accvgpr_write_b32 a{i}, 0', [], [f'a{i}'])
        # ring fill: K(b+2) V(b) for b = 0 .. R-3 (block b of K in slot b, of V in slot b). The kernel issued the
        # head (K0, K1, a zero V(-1) in slot R-1) before its Q loads, and this wavefront's part of it has landed
        # (vmcnt(0) above); the barrier makes every wavefront's part visible.
        for b in range(R - 2):
            self.dma_k(e, b + 2)
            e.raw(f's_cmp_eq_u32 %[nbak], {b + 3}')
            e.raw(f's_cselect_b64 s[{KRES}:{KRES + 1}], s[{SKSW}:{SKSW + 1}], s[{KRES}:{KRES + 1}]')
            self.dma_v(e, b)
            e.raw(f's_cmp_eq_u32 s{SVTHR}, {(b + 1 - (R - 2)) & 0xffffffff}')
            e.raw(f's_cbranch_scc0 .Lvf{b}_%=')
            for line in v_advance(R):
                e.raw(line)
            e.label(f'.Lvf{b}_%=')
        # the value events up to block R - 2 are taken: s84 is now at least 1 (or never)
        e.raw(f's_sub_u32 s{SNB1}, %[nb], 1')
        e.raw(f's_min_u32 s{SNB1}, s{SNB1}, s{SVTHR}')
        e.raw(f's_min_u32 s{SNB1}, s{SNB1}, s{SKTHR}')
        e.raw('s_barrier')
        # a wavefront whose 64 queries all lie past the segment only keeps up the block's K/V stream
        e.raw('s_cmp_eq_u32 %[dead], 0')
        e.raw('s_cbranch_scc0 .Ldead_%=')
        # S(0) = K(0) Q^T (no offset yet); the operands of iteration 0's steps 0..3 (K(1), V(-1)) are read behind it
        for k in range(8):
            self.read_k(e, k, 0)
        pre = [('k', k, 1) if t == 0 else ('v', k, R - 1) for k in range(4) for t in range(2)]
        for k in range(8):
            for qb in range(2):
                self.mfma_s(e, 0, qb, k, seed='0')
            if 1 <= k <= 4:
                # K operand k-1 is consumed by both query blocks: its register can take iteration 0's step k-1
                for _ in range(2):
                    kind, kk, slot = pre.pop(0)
                    (self.read_k if kind == 'k' else self.read_v)(e, kk, slot)
        # m = block 0's maximum (after the mask when block 0 is the last one); S(0) -= m; the -m seed of later blocks
        e.nop_to(MFMA_WAIT)
        e.raw(f's_cmp_eq_u32 s{SNB1}, 0')
        e.raw('s_cbranch_scc0 .Lpmask_%=')
        self.mask(e, 0)
        e.label('.Lpmask_%=')
        for qb in range(2):
            self.row_max(e, 0, qb, M0 + qb, A0)
            for r in range(16):
                e.valu(f'v_sub_f32_e32 v{S(0, qb, r)}, v{S(0, qb, r)}, v{M0 + qb}', [v(S(0, qb, r)), v(M0 + qb)],
                       [v(S(0, qb, r))])
                e.valu(f'v_sub_f32_e32 v{MCV(qb) + r}, 0, v{M0 + qb}', [v(M0 + qb)], [v(MCV(qb) + r)])

    def dead_loop(self):
        """the key loop of a wavefront without live queries: per iteration only the barrier and its share of the
        K/V refill, the same as a body's, so that the block's barriers and LDS DMA stay in step; no MFMA, softmax or
        LDS read. Exits to the end of the asm block once every DMA has landed, with the next item's Q loads issued
        (no output is written)."""
        R = self.R
        lines = ['.Ldead_%=:']
        for J in range(R):
            lines.append(f's_waitcnt vmcnt({4 * (R - 3)})')
            lines.append('s_barrier')
            for op in self.dma_ops(J):
                lines.append(op[1])
                if op[0] == 'm0':
                    lines.append('s_nop 0')          # an SALU write of M0 and the LDS DMA reading it
            lines += [f's_add_u32 s{SJ}, s{SJ}, 1', f's_cmp_eq_u32 s{SJ}, s{SVTHR}',
                      f's_cbranch_scc0 .Ldvn{J}_%='] + v_advance(R) + [f'.Ldvn{J}_%=:',
                      f's_cmp_eq_u32 s{SJ}, s{SKTHR}',
                      f's_cselect_b64 s[{KRES}:{KRES + 1}], s[{SKSW}:{SKSW + 1}], s[{KRES}:{KRES + 1}]',
                      f's_cmp_ge_u32 s{SJ}, %[nb]', 's_cbranch_scc1 .Ldeadexit_%=']
        lines += ['s_branch .Ldead_%=', '.Ldeadexit_%=:'] + self.q_prefetch()
        lines += ['s_waitcnt vmcnt(16)', 's_branch .Ldone_%=']
        return lines

    def generate(self):
        R = self.R
        e = Emitter()
        self.prologue(e)
        pro_lines = list(e.lines)
        # the prologue leaves the same prefetched reads outstanding as a body's phase B, in the same order
        state = (dict(e.mfma_w), dict(e.valu_w), e.pos, list(e.lds))
        # bodies: run the whole ring twice so that body 0 sees the wrap-around hazards of body R-1
        for attempt in range(2):
            e2 = Emitter()
            mw, vw, pos, lds = state
            e2.mfma_w = {r: p - pos for r, p in mw.items()}
            e2.valu_w = {r: p - pos for r, p in vw.items()}
            e2.lds = [set(x) for x in lds]
            e2.label('.Lloop_%=')
            for J in range(R):
                self.body(e2, J)
            e2.raw('s_branch .Lloop_%=')
            if attempt == 0:
                mw2 = {r: p - e.pos for r, p in e.mfma_w.items()}
                vw2 = {r: p - e.pos for r, p in e.valu_w.items()}
                for r, p in e2.mfma_w.items():
                    mw2[r] = max(mw2.get(r, -10 ** 9), p - e2.pos)
                for r, p in e2.valu_w.items():
                    vw2[r] = max(vw2.get(r, -10 ** 9), p - e2.pos)
                state = (mw2, vw2, 0, lds)
        lines = pro_lines + e2.lines
        for J in range(R):
            lines += [f'.Lexit{J}_%=:', f's_mov_b32 s{SVOFF}, {J * SLOT}', f's_branch .Lepi{J & 1}_%=']
        for J in range(R):
            lines += self.end_block(J)
        for J in range(R):
            lines += self.mask_block(J)
        for par in range(2):
            lines += self.rescale_block(par)
        for par in range(2):
            lines += self.epilogue(par)
        lines += self.dead_loop()
        lines += self.store_block()
        # no scalar load of the value events may land after the block: its registers are the compiler's again
        lines += ['.Ldone_%=:', 's_waitcnt lgkmcnt(0)']
        return lines


def render(ring):
    k = Kernel(ring)
    lines = k.generate()
    body = '\n'.join(f'  "{l}\\n\\t"' if not l.endswith(':') else f'  "{l}\\n"' for l in lines)
    clob = ', '.join(f'"v{i}"' for i in range(FIRST_FIXED, 256)) + ', ' + ', '.join(f'"a{i}"' for i in range(192))
    clob += ', ' + ', '.join(f'"s{i}"' for i in range(64, LAST_SGPR + 1)) + ', "vcc", "scc", "memory"'
    qload = ' \\\n  '.join(f'"{l}\\n\\t"' for l in Kernel.q_prefetch())
    qclob = ', '.join(f'"a{i}"' for i in range(128, 192))
    cases = []
    for qb in range(2):
        for k in range(8):
            # the first step waits until earlier loads into these registers (a key loop's exit) have landed
            w = 's_waitcnt vmcnt(0)\\n\\t' if qb == k == 0 else ''
            w += ''.join(f'v_accvgpr_write_b32 a{QA(qb, k) + i}, %{i}\\n\\t' for i in range(4))
            cl = ', '.join(f'"a{QA(qb, k) + i}"' for i in range(4))
            cases.append(f'case {8 * qb + k}: asm volatile("{w}" :: "v"((x)[0]), "v"((x)[1]), "v"((x)[2]), '
                         f'"v"((x)[3]) : {cl}); break;')
    qset = ' \\\n    '.join(cases)
    hdr = f'''// Generated by gen_attn_ring64.py (ring of {ring} K and {ring} V slots): do not edit.
// The key loop of attn8_kernel; operands and fixed registers are described in the generator.
#define ONEREEL_RING64 {ring}
#define ONEREEL_RING64_ASM \\
{body.replace(chr(10), " " + chr(92) + chr(10))}
#define ONEREEL_RING64_CLOBBERS {clob}
// an item's queries into the key loop's registers a128..a191 (query block qb, k-step k at a[128 + 32 qb + 4 k : +3]):
// loaded from the lane's two rows (%[qa0], %[qa1]), or written from four dwords x[0..3] per (qb, k) (qb and k
// compile-time constants)
#define ONEREEL_RING64_QLOAD {qload}
#define ONEREEL_RING64_QCLOBBERS {qclob}
#define ONEREEL_RING64_QSET_STEP(qb, k, x) \\
  do {{ \\
    switch (8 * (qb) + (k)) {{ \\
    {qset} \\
    }} \\
  }} while (0)
'''
    return hdr


if __name__ == '__main__':
    ap = argparse.ArgumentParser()
    ap.add_argument('--ring', type=int, default=8)
    ap.add_argument('--out', default=str(Path(__file__).resolve().parent / 'attn_ring64.inc'))
    a = ap.parse_args()
    Path(a.out).write_text(render(a.ring))
    print(a.out)
