#!/usr/bin/env python3
"""Writes dkdv64_item.inc: the instruction stream of one 128-row stage of the D = 64
dK/dV pass (fa_bwd_dkdv64.hip) for one wave, as the text of one inline-asm statement.

Why a generated schedule: per 32-row query block a wave issues 16 MFMAs (S and dP, then
dV and dK), 32 LDS operand reads and 64 VALU operations (exp2, the dS products, bf16
packing).  The compiler's schedule runs a block's phases one after another (products,
then all exponentials, then products), so half of the MFMAs have no VALU work beside them,
and it waits on each LDS read right before its consumer.  Here the four blocks of a stage
form a software pipeline: round i runs block i's softmax on the VALU under block i-1's
dV/dK products and block i+1's S/dP products (two register sets, alternating), and every
LDS read is issued a few products ahead of its use.

The generator also does what the compiler's hazard recognizer and waitcnt insertion would
do, since neither looks inside an asm statement:
  * s_waitcnt lgkmcnt(n) before the first instruction that touches a register an LDS read
    is still filling (LDS reads complete in order, so n counts the younger reads);
  * s_nop padding for the gfx950 dependencies that hardware does not interlock:
    MFMA (8 passes) result -> VALU or LDS access: 12 wait states; VALU result -> MFMA
    operand: 2; transcendental result -> VALU: 1.  An MFMA chain on the same accumulator
    needs none.  The statement starts with s_nop 1, since the compiler's code just before
    it may have written an MFMA operand.

Register map inside the statement (fixed, so sub-ranges of a result can be named; the
statement clobbers v[0:111]):
  v[0:15] S of register set 0, v[16:31] its dP (then dS), v[32:63] the same for set 1;
  P (and dS) are packed to bf16 in place, rows 8m..8m+7 into registers 8m..8m+3;
  v[64:79] Q row fragments (k-step kk at v[64+4kk]), v[80:95] dO row fragments, v[96:103]
  dO^T fragments (db = 0, 1), v[104:111] Q^T fragments.
Operands: %0, %1 the dK^T accumulators (db = 0, 1), %2, %3 the dV^T ones, %4..%7 the K
fragments (k-step kk), %8..%11 the V fragments, all in AGPRs; then the LDS byte addresses
aR0..aR3 (row reads, k-step kk), aT (transposed reads: column block db = 0, 1 times row
half h = 0, 1), aN (-LSE/scale rows), the SGPR scale*log2(e), the lane's lq - 4lg (the
diagonal mask) and the SGPR mode that picks the variant.

Rows past T need no mask: their Q, dO, LSE and Delta read as zero, so P = 1 and dS = 0
there and their dV, dK contributions are exact zeros.

usage: python gen_dkdv64_asm.py [out.inc]
"""
import os
import sys

MFMA_RESULT_WS = 12   # 8-pass XDL write -> VALU / LDS access of the same register
VALU_TO_MFMA_WS = 2   # VALU write -> MFMA operand read
TRANS_TO_VALU_WS = 1  # v_exp write -> VALU read
MAX_LGKM = 15         # s_waitcnt lgkmcnt field width
# A register an MFMA reads as an A or B operand is refilled by an LDS read only after
# WAR_MFMAS more MFMAs of the wave have issued (a margin: the hardware reads those operands
# when the product starts, and a refill right behind the product has not been needed).
WAR_MFMAS = 2

# LDS stage layout (bytes from the stage base): the Q tile (STAGE_ROWS rows of 128 bytes),
# the dO tile, then -LSE/scale and -Delta for the stage's rows (fp32); the row addresses
# carry the stage base, the init address carries the base of the -LSE/scale rows
STAGE_ROWS = 128
DO_OFF = STAGE_ROWS * 128
ND_OFF = STAGE_ROWS * 4

# register bases
S = [0, 32]      # S of block b
P = [16, 48]     # dP / dS of block b
QA, DA, DOT, QT = 64, 80, 96, 104
N_VTEMP = 112   # v[0:111]

# operand numbers of the asm statement (see dkdv64_stage in fa_bwd_dkdv64.hip)
OP_DK = [0, 1]              # dK^T accumulators (AGPR), column block db
OP_DV = [2, 3]              # dV^T accumulators (AGPR)
OP_KF = [4, 5, 6, 7]        # K fragments (AGPR), k-step kk
OP_VF = [8, 9, 10, 11]      # V fragments (AGPR)
OP_AR = [12, 13, 14, 15]    # row-fragment reads, k-step kk
OP_AT = [[16, 17], [18, 19]]  # transposed reads, [column block db][row half h]
OP_AN = 20
OP_SCALE = 21
OP_DL = 22       # VGPR: lq - 4lg (diagonal mask)
OP_MODE = 23     # SGPR: 0 = FULL, 1 + w = DIAG<w>


def vr(b, n):
    return [f'v{b + i}' for i in range(n)]


def vt(b, n):
    return f'v[{b}:{b + n - 1}]' if n > 1 else f'v{b}'


class Op:
    def __init__(self, text, kind, reads=(), writes=(), tag=''):
        self.text, self.kind, self.reads, self.writes, self.tag = text, kind, list(reads), list(writes), tag


class Emitter:
    def __init__(self):
        self.lines = []
        self.ws = 0              # wait states issued so far
        self.last = {}           # reg -> (ws after the writer issued, writer kind)
        self.lds = []            # outstanding LDS reads: sets of registers they fill
        self.n_nops = 0
        self.n_waits = 0
        self.n_mfma = 0
        self.mfma_read = {}      # reg -> MFMA count when an MFMA last read it

    def _wait_lds(self, regs):
        hit = -1
        for i, w in enumerate(self.lds):
            if w & regs:
                hit = i
        if hit >= 0:
            n = len(self.lds) - hit - 1
            self.lines.append(f's_waitcnt lgkmcnt({n})')
            self.lds = self.lds[hit + 1:]
            self.ws += 1
            self.n_waits += 1

    def _need(self, op):
        need = 0
        for r in op.reads + op.writes:
            if r not in self.last:
                continue
            at_ws, kind = self.last[r]
            gap = self.ws - at_ws
            req = 0
            if kind == 'mfma' and op.kind in ('valu', 'trans', 'lds'):
                req = MFMA_RESULT_WS
            elif kind == 'mfma' and op.kind == 'mfma':
                # chains (srcC/vdst = the previous vdst) need nothing; any other use of a
                # product's result as an operand is not part of this schedule
                if r not in op.writes:
                    req = MFMA_RESULT_WS
            elif kind in ('valu', 'trans') and op.kind == 'mfma':
                req = VALU_TO_MFMA_WS
            elif kind == 'trans' and op.kind in ('valu', 'trans'):
                req = TRANS_TO_VALU_WS
            need = max(need, req - gap)
        return need

    def emit(self, op):
        regs = set(op.reads) | set(op.writes)
        self._wait_lds(regs)
        if op.kind == 'lds' and len(self.lds) >= MAX_LGKM:
            self.lines.append(f's_waitcnt lgkmcnt({MAX_LGKM - 1})')
            self.lds = self.lds[len(self.lds) - (MAX_LGKM - 1):]
            self.ws += 1
            self.n_waits += 1
        if op.kind == 'lds':
            for r in op.writes:
                if r in self.mfma_read and self.n_mfma - self.mfma_read[r] < WAR_MFMAS:
                    raise SystemExit(f'WAR: {op.text} overwrites {r} of an MFMA that may not have started')
        need = self._need(op)
        while need > 0:
            k = min(need, 16)
            self.lines.append(f's_nop {k - 1}')
            self.ws += k
            need -= k
            self.n_nops += k
        self.lines.append(op.text)
        self.ws += 1
        if op.kind == 'mfma':
            self.n_mfma += 1
            for r in op.reads:
                if r not in op.writes:
                    self.mfma_read[r] = self.n_mfma
        for r in op.writes:
            self.last[r] = (self.ws, op.kind)
        if op.kind == 'lds':
            self.lds.append(set(op.writes))

    def finish(self):
        if self.lds:
            self.lines.append('s_waitcnt lgkmcnt(0)')
            self.lds = []
        # the accumulators' last products may still run: the statement ends with the
        # wait states a following VALU access of their registers would need
        pend = min((self.ws - w for w, k in self.last.values() if k == 'mfma'), default=99)
        if pend < MFMA_RESULT_WS:
            k = MFMA_RESULT_WS - pend
            self.lines.append(f's_nop {k - 1}')
            self.n_nops += k


# ---------------------------------------------------------------- operations
# rb: register block (which S/dP register set), lb: LDS block (query rows 32lb.. of the item)
def l_rows(lb, kk, tensor):
    """Q (tensor 0) or dO (tensor 1) row fragment of k-step kk, LDS block lb."""
    dst = (QA if tensor == 0 else DA) + 4 * kk
    off = DO_OFF * tensor + 4096 * lb
    return Op(f'ds_read_b128 {vt(dst, 4)}, %{OP_AR[kk]} offset:{off}', 'lds', writes=vr(dst, 4))


def l_init(rb, lb, a, which):
    """-LSE/scale (which 0, into S) or -Delta (which 1, into dP) rows 8a+4lg.. of LDS
    block lb."""
    dst = (S[rb] if which == 0 else P[rb]) + 4 * a
    off = ND_OFF * which + 128 * lb + 32 * a
    return Op(f'ds_read_b128 {vt(dst, 4)}, %{OP_AN} offset:{off}', 'lds', writes=vr(dst, 4))


def l_tr(lb, m, db, tensor, h):
    """Half h of the transposed fragment (query rows 32lb+16m.., columns 32db..) of Q
    (tensor 0, -> Q^T registers) or dO (tensor 1, -> dO^T registers)."""
    dst = (QT if tensor == 0 else DOT) + 4 * db + 2 * h
    off = DO_OFF * tensor + (32 * lb + 16 * m) * 128
    return Op(f'ds_read_b64_tr_b16 {vt(dst, 2)}, %{OP_AT[db][h]} offset:{off}', 'lds', writes=vr(dst, 2))


def l_tr_set(lb, m, tensor):
    return [l_tr(lb, m, db, tensor, h) for db in range(2) for h in range(2)]


def m_s(rb, kk):
    return Op(f'v_mfma_f32_32x32x16_bf16 {vt(S[rb], 16)}, {vt(QA + 4 * kk, 4)}, %{OP_KF[kk]}, {vt(S[rb], 16)}',
              'mfma', reads=vr(S[rb], 16) + vr(QA + 4 * kk, 4), writes=vr(S[rb], 16))


def m_p(rb, kk):
    return Op(f'v_mfma_f32_32x32x16_bf16 {vt(P[rb], 16)}, {vt(DA + 4 * kk, 4)}, %{OP_VF[kk]}, {vt(P[rb], 16)}',
              'mfma', reads=vr(P[rb], 16) + vr(DA + 4 * kk, 4), writes=vr(P[rb], 16))


def m_dv(rb, m, db):
    acc = f'%{OP_DV[db]}'
    return Op(f'v_mfma_f32_32x32x16_bf16 {acc}, {vt(DOT + 4 * db, 4)}, {vt(S[rb] + 8 * m, 4)}, {acc}',
              'mfma', reads=vr(DOT + 4 * db, 4) + vr(S[rb] + 8 * m, 4) + [acc], writes=[acc])


def m_dk(rb, m, db):
    acc = f'%{OP_DK[db]}'
    return Op(f'v_mfma_f32_32x32x16_bf16 {acc}, {vt(QT + 4 * db, 4)}, {vt(P[rb] + 8 * m, 4)}, {acc}',
              'mfma', reads=vr(QT + 4 * db, 4) + vr(P[rb] + 8 * m, 4) + [acc], writes=[acc])


def dvdk(rb, m):
    """The four products of row group m (16 query rows): dV^T, dK^T for both column blocks,
    the two dV products first (they free the dO^T registers), then the two dK ones."""
    return [m_dv(rb, m, 0), m_dv(rb, m, 1), m_dk(rb, m, 0), m_dk(rb, m, 1)]


def softmax(rb, diag):
    """P = exp2(S' * scale*log2e) and dS = P * (dP - Delta) in place, then both packed to
    bf16 in place; element pairs are interleaved so no step waits on the previous one.
    diag: the block's rows start at the wave's first key, and score (row 8(r/4)+4lg+r%4,
    key lq) is masked (P = 0) when lq - 4lg > 8(r/4) + r%4, i.e. key > row."""
    ops = []
    s, p = S[rb], P[rb]
    for m in range(2):
        for r0 in range(8 * m, 8 * m + 8, 2):
            for r in (r0, r0 + 1):
                ops.append(Op(f'v_mul_f32 v{s + r}, %{OP_SCALE}, v{s + r}', 'valu', reads=[f'v{s + r}'], writes=[f'v{s + r}']))
            for r in (r0, r0 + 1):
                ops.append(Op(f'v_exp_f32 v{s + r}, v{s + r}', 'trans', reads=[f'v{s + r}'], writes=[f'v{s + r}']))
            if diag:  # P = exp2(-inf) = +0 for the masked scores, as in the unscheduled code
                for r in (r0, r0 + 1):
                    t = 8 * (r >> 2) + (r & 3)
                    ops.append(Op(f'v_cmp_lt_i32 vcc, {t}, %{OP_DL}', 'valu', reads=[], writes=['vcc']))
                    ops.append(Op(f'v_cndmask_b32_e64 v{s + r}, v{s + r}, 0, vcc', 'valu',
                                  reads=[f'v{s + r}', 'vcc'], writes=[f'v{s + r}']))
            for r in (r0, r0 + 1):
                ops.append(Op(f'v_mul_f32 v{p + r}, v{s + r}, v{p + r}', 'valu', reads=[f'v{s + r}', f'v{p + r}'], writes=[f'v{p + r}']))
        for base in (s, p):
            for j in range(4):
                src0, src1 = base + 8 * m + 2 * j, base + 8 * m + 2 * j + 1
                ops.append(Op(f'v_cvt_pk_bf16_f32 v{base + 8 * m + j}, v{src0}, v{src1}', 'valu',
                              reads=[f'v{src0}', f'v{src1}'], writes=[f'v{base + 8 * m + j}']))
    return ops


def spread(mfmas, fillers, counts):
    """MFMA i followed by counts[i] filler operations (the rest after the last)."""
    out, k = [], 0
    for i, m in enumerate(mfmas):
        out.append(m)
        c = counts[i] if i < len(counts) else 0
        out.extend(fillers[k:k + c])
        k += c
    out.extend(fillers[k:])
    return out


def even(n_fill, n_mfma):
    base, extra = divmod(n_fill, n_mfma)
    return [base + (1 if i < extra else 0) for i in range(n_mfma)]


LDS_LEAD = 3  # MFMAs between an LDS read and its first consumer, where registers allow


def hoist_lds(ops, lead=LDS_LEAD):
    """Places the LDS reads of an op list.  Each read goes LDS_LEAD MFMAs ahead of its
    first consumer (the first later instruction that uses a register it fills), or as
    early as the registers allow if that is later: after the last instruction that still
    uses their previous value, and after the writer of any register it reads (an address).
    Reads placed at the same point keep consumer order."""
    core = [op for op in ops if op.kind != 'lds']
    index = {id(op): i for i, op in enumerate(core)}
    placed = []  # (position in core: insert before core[pos], consumer index, seq, op)
    n_before = 0  # core ops listed before the current LDS op
    for seq, op in enumerate(ops):
        if op.kind != 'lds':
            n_before += 1
            continue
        dst, src = set(op.writes), set(op.reads)
        legal = 0
        for i in range(n_before - 1, -1, -1):
            c = core[i]
            if dst & (set(c.reads) | set(c.writes)) or src & set(c.writes):
                legal = i + 1
                if c.kind == 'mfma' and dst & set(c.reads):
                    # WAR_MFMAS more MFMAs must issue first
                    seen = 0
                    while legal < len(core) and seen < WAR_MFMAS:
                        if core[legal].kind == 'mfma':
                            seen += 1
                        legal += 1
                break
        cons = len(core)
        for i in range(n_before, len(core)):
            c = core[i]
            if dst & (set(c.reads) | set(c.writes)):
                cons = i
                break
        if legal > cons:
            raise SystemExit(f'LDS read {op.text} cannot go before its consumer {core[cons].text}: '
                             'the registers it fills are still in use there')
        want, need = cons, lead
        while need > 0 and want > legal:
            want -= 1
            if core[want].kind == 'mfma':
                need -= 1
        placed.append((max(legal, want), cons, seq, op))
    placed.sort(key=lambda t: (t[0], t[1], t[2]))
    out, k = [], 0
    for i, c in enumerate(core + [None]):
        while k < len(placed) and placed[k][0] == i:
            out.append(placed[k][3])
            k += 1
        if c is not None:
            out.append(c)
    return out


def schedule_stage(blocks):
    """A software pipeline over the 32-row blocks of one LDS stage.  blocks: list of
    (lds block, diagonal) in order; block i uses register set i % 2.  Round i runs block
    i's softmax on the VALU under two MFMA groups: block i-1's dV/dK products (which free
    the other register set and the transposed-fragment registers), then block i+1's S/dP
    products into that set.  Block 0's S/dP come first on their own, the last block's
    dV/dK last.  LDS reads are listed where their registers are free and then hoisted."""
    n = len(blocks)
    ops = []
    lb0 = blocks[0][0]
    ops += [l_init(0, lb0, a, 0) for a in range(4)] + [l_rows(lb0, 0, 0)]
    ops += [l_init(0, lb0, a, 1) for a in range(4)] + [l_rows(lb0, 0, 1)]
    for kk in range(1, 4):
        ops += [l_rows(lb0, kk, 0), l_rows(lb0, kk, 1)]
    for kk in range(4):
        ops += [m_s(0, kk), m_p(0, kk)]
    if n > 1:
        lb1 = blocks[1][0]
        ops += [l_rows(lb1, kk, t) for kk in range(4) for t in (0, 1)]
        ops += [l_init(1, lb1, a, w) for w in range(2) for a in range(4)]
    for i in range(n):
        lb, diag = blocks[i]
        rs, os_ = i % 2, 1 - i % 2
        sm = softmax(rs, diag)
        mf = []
        if i >= 1:
            plb = blocks[i - 1][0]
            # block i-1's dV/dK: dK (reads dS in the P set) before dV (P in the S set),
            # so the P set frees first; the m = 1 fragments load as m = 0's products issue
            mf += [m_dk(os_, 0, 0), m_dk(os_, 0, 1), ('L', l_tr_set(plb, 1, 0)),
                   m_dv(os_, 0, 0), m_dv(os_, 0, 1), ('L', l_tr_set(plb, 1, 1)),
                   m_dk(os_, 1, 0), m_dk(os_, 1, 1), m_dv(os_, 1, 0), m_dv(os_, 1, 1)]
        if i + 1 < n:
            nlb = blocks[i + 1][0]
            if i >= 1:
                mf.append(('L', [l_rows(nlb, kk, t) for kk in range(4) for t in (0, 1)] +
                           [l_init(os_, nlb, a, w) for w in (1, 0) for a in range(4)]))
            mf += [m_p(os_, 0), m_p(os_, 1), m_s(os_, 0), m_p(os_, 2), m_s(os_, 1), m_p(os_, 3),
                   m_s(os_, 2), m_s(os_, 3)]
        # block i's m = 0 transposed fragments, for its dV/dK in the next round
        mf.append(('L', l_tr_set(lb, 0, 1) + l_tr_set(lb, 0, 0)))
        n_m = sum(1 for x in mf if not isinstance(x, tuple))
        per = even(len(sm), max(n_m, 1))
        k = j = 0
        for x in mf:
            if isinstance(x, tuple):
                ops += x[1]
                continue
            ops.append(x)
            ops += sm[k:k + per[j]]
            k += per[j]
            j += 1
        ops += sm[k:]
    # the last block's dV/dK
    llb = blocks[-1][0]
    ls = (n - 1) % 2
    ops += [m_dk(ls, 0, 0), m_dk(ls, 0, 1)] + l_tr_set(llb, 1, 0) + [m_dv(ls, 0, 0), m_dv(ls, 0, 1)] + \
        l_tr_set(llb, 1, 1) + [m_dk(ls, 1, 0), m_dk(ls, 1, 1), m_dv(ls, 1, 0), m_dv(ls, 1, 1)]
    return hoist_lds(ops)


# One variant per case of a 128-row stage against a wave's 32 keys: every block below
# the diagonal, or (the stage that holds the diagonal) wave w's blocks from w on, block w
# on the diagonal.  Rows past T need no case of their own.
VARIANTS = {
    'FULL': ([(b, False) for b in range(4)], 'all four 32-row blocks below the diagonal'),
}
for _w in range(4):
    VARIANTS[f'DIAG{_w}'] = ([(_w, True)] + [(b, False) for b in range(_w + 1, 4)],
                             f'blocks {_w}..3 of the diagonal stage for wave {_w}')


def generate(ops):
    e = Emitter()
    e.lines.append('s_waitcnt lgkmcnt(0)')
    for op in ops:
        e.emit(op)
    e.finish()
    return e


DEFAULT_OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'dkdv64_item.inc')


def render(verbose=False):
    """The text of dkdv64_item.inc."""
    # One statement holds every variant behind a branch on the mode operand, so the
    # compiler sees a single asm site (two sites with the same operands make it keep
    # extra copies of them).  Labels are made unique per expansion with %=.
    names = list(VARIANTS)
    text = ['// Generated by gen_dkdv64_asm.py (do not edit): the instruction streams of one 128-row\n'
            '// stage of the D = 64 dK/dV pass for one wave, one per causal-mask case, selected by\n'
            '// the mode operand (0: FULL, 1 + w: DIAG<w>).\n']
    # s_nop 1 first: the compiler's code right before may have written an MFMA operand
    # (a VALU result needs 2 wait states before an MFMA reads it)
    lines = ['s_nop 1']
    for i, name in enumerate(names[1:], 1):
        lines += [f's_cmp_eq_u32 %{OP_MODE}, {i}', f's_cbranch_scc1 .Ldkv_{name}_%=']
    for i, name in enumerate(names):
        blocks, desc = VARIANTS[name]
        e = generate(schedule_stage(blocks))
        n_mfma = sum(1 for l in e.lines if l.startswith('v_mfma'))
        n_lds = sum(1 for l in e.lines if l.startswith('ds_'))
        n_valu = sum(1 for l in e.lines if l.startswith('v_') and not l.startswith('v_mfma'))
        text.append(f'// {name}: {desc}; {n_mfma} MFMA, {n_lds} LDS reads, {n_valu} VALU, '
                    f'{e.n_waits} lgkmcnt waits, {e.n_nops} nop wait states.\n')
        if verbose:
            print(f'{name}: {n_mfma} MFMA, {n_lds} LDS, {n_valu} VALU, {e.n_waits} waits, {e.n_nops} nops')
        if i > 0:
            lines.append(f'.Ldkv_{name}_%=:')
        lines += e.lines
        if i < len(names) - 1:
            lines.append('s_branch .Ldkv_end_%=')
    lines.append('.Ldkv_end_%=:')
    body = ''.join(f'  "{l}\\n"\n' for l in lines)
    text.append('#define TTFA_DKDV64_STAGE_ASM \\\n' + body.rstrip('\n').replace('\n', ' \\\n') + '\n')
    clob = ', '.join(f'"v{i}"' for i in range(N_VTEMP))
    text.append(f'\n#define TTFA_DKDV64_ITEM_CLOBBERS {clob}, "vcc", "scc"\n')
    return ''.join(text)


def main():
    out = sys.argv[1] if len(sys.argv) > 1 else DEFAULT_OUT
    with open(out, 'w') as f:
        f.write(render(verbose=True))
    print(f'wrote {out}')


if __name__ == '__main__':
    main()
