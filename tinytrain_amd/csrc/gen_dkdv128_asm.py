#!/usr/bin/env python3
"""Writes dkdv128_item.inc: the instruction stream of one 128-row stage of the D = 128
dK/dV pass (fa_bwd_dkdv128.hip) for one wave (32 keys), as the text of one inline-asm
statement.

The pass runs one wave per SIMD (the dK/dV accumulators and the K/V fragments take 192
AGPRs), so no other wave can issue VALU work while a wave's products run: the compiler's
schedule (products, then all exponentials, then products) leaves the matrix cores idle
through every softmax.  Here, as in the D = 64 pass (gen_dkdv64_asm.py, whose emitter and
LDS placement this reuses), the four 32-row blocks of a stage form a software pipeline:
round i runs block i's exponentials and dS on the VALU under block i-1's dV/dK products
and block i+1's S/dP products, in two alternating register sets.  At D = 128 a block has
32 products (S and dP over 8 k-steps, dV and dK over 4 column blocks x 2 row groups)
against ~70 VALU operations, so the VALU work hides entirely.

Register map (fixed; the statement clobbers v[0:159]):
  v[0:15] S of register set 0, v[16:31] its dP (then dS), v[32:63] set 1; P and dS are
  packed to bf16 in place, rows 8m..8m+7 into registers 8m..8m+3;
  v[64:95] Q row fragments (k-step kk at v[64+4kk]), v[96:127] dO row fragments,
  v[128:143] dO^T fragments (column block db at +4db), v[144:159] Q^T fragments.
Operands: %0..%3 the dK^T accumulators (column blocks db), %4..%7 the dV^T ones,
%8..%15 the K fragments (k-step kk), %16..%23 the V fragments, all in AGPRs; %24..%31 the
LDS byte addresses of the row-fragment reads per k-step, %32..%39 those of the transposed
reads (column block db, half h at %32+2db+h), %40 the -LSE/scale rows' address, %41 the
SGPR scale*log2(e), %42 lq - 4lg (the diagonal mask), %43 the SGPR mode (0: FULL,
1 + w: DIAG<w>).  The tiles use swz_rows128, whose XOR takes row bits 0-3 into all four
chunk bits (a row read's 16 rows hit 16 distinct bank groups), so every k-step and every
8-row half has an address of its own; the 32-row blocks (+8192 bytes), the dO tile
(+32768) and the 16-row groups of the transposed reads (+4096) are constant offsets.

usage: python gen_dkdv128_asm.py [out.inc]
"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import gen_dkdv64_asm as g  # noqa: E402  (emitter, LDS placement, helpers)

Op, vr, vt = g.Op, g.vr, g.vt

D = 128
KK = D // 16          # k-steps of S and dP
DB = D // 32          # column blocks of dK^T / dV^T
ROW_BYTES = D * 2
STAGE_ROWS = 128
DO_OFF = STAGE_ROWS * ROW_BYTES   # dO tile after the Q tile (bytes)
ND_OFF = STAGE_ROWS * 4           # -Delta rows after the -LSE/scale rows (bytes)
BLOCK_BYTES = 32 * ROW_BYTES

S = [0, 32]
P = [16, 48]
QA, DA, DOT, QT = 64, 96, 128, 144
N_VTEMP = 160

OP_DK = [0, 1, 2, 3]
OP_DV = [4, 5, 6, 7]
OP_KF = list(range(8, 16))
OP_VF = list(range(16, 24))
OP_AR = list(range(24, 32))  # row-fragment reads, k-step kk
OP_AT = list(range(32, 40))  # transposed reads, column block db, half h: 2db + h
OP_AN = 40
OP_SCALE = 41
OP_DL = 42
OP_MODE = 43


def l_rows(lb, kk, tensor):
    """Q (tensor 0) or dO (tensor 1) row fragment of k-step kk, LDS block lb."""
    dst = (QA if tensor == 0 else DA) + 4 * kk
    off = DO_OFF * tensor + BLOCK_BYTES * lb
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
    off = DO_OFF * tensor + (32 * lb + 16 * m) * ROW_BYTES
    return Op(f'ds_read_b64_tr_b16 {vt(dst, 2)}, %{OP_AT[2 * db + h]} offset:{off}', 'lds', writes=vr(dst, 2))


def l_tr_set(lb, m, tensor):
    return [l_tr(lb, m, db, tensor, h) for db in range(DB) for h in range(2)]


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


def softmax(rb, diag):
    """P = exp2(S' * scale*log2e) and dS = P * (dP - Delta) in place, then both packed to
    bf16 in place (the steps of the D = 64 stream; they do not depend on D).  diag: the
    block's rows start at the wave's first key, and score (row 8(r/4)+4lg+r%4, key lq)
    is masked (P = 0) when lq - 4lg > 8(r/4) + r%4, i.e. key > row."""
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


def sdp_products(rs):
    """A block's S and dP products, the two chains interleaved (no product waits on the
    one just before it).  The dP chain starts two products ahead: the register set's
    -LSE/scale rows (the S chain's initial value) may only be refilled two products after
    the previous block's last dV product read that set's packed P."""
    order = [m_p(rs, 0), m_p(rs, 1)]
    for kk in range(KK):
        order.append(m_s(rs, kk))
        if kk + 2 < KK:
            order.append(m_p(rs, kk + 2))
    return order


def dvdk_group(rs, m):
    """Row group m's dK and dV products over the column blocks: dK (reads dS in the P
    set) first, so the P set frees first."""
    return [m_dk(rs, m, db) for db in range(DB)] + [m_dv(rs, m, db) for db in range(DB)]


def schedule_stage(blocks):
    """A software pipeline over the 32-row blocks of one LDS stage.  blocks: list of
    (lds block, diagonal); block i uses register set i % 2.  Round i runs block i's
    softmax on the VALU under block i-1's dK/dV products and block i+1's S/dP products.
    LDS reads are listed where their registers are free and then hoisted."""
    n = len(blocks)
    ops = []
    lb0 = blocks[0][0]
    ops += [l_init(0, lb0, a, w) for w in range(2) for a in range(4)]
    ops += [l_rows(lb0, kk, t) for kk in range(KK) for t in (0, 1)]
    ops += sdp_products(0)
    if n > 1:
        lb1 = blocks[1][0]
        ops += [l_rows(lb1, kk, t) for kk in range(KK) for t in (0, 1)]
        ops += [l_init(1, lb1, a, w) for w in range(2) for a in range(4)]
    for i in range(n):
        lb, diag = blocks[i]
        rs, os_ = i % 2, 1 - i % 2
        sm = softmax(rs, diag)
        mf = []
        if i >= 1:
            plb = blocks[i - 1][0]
            # block i-1's dK/dV: row group 0, then its m = 1 transposed fragments as row
            # group 0's products free the registers, then row group 1
            mf += dvdk_group(os_, 0)
            mf.append(('L', l_tr_set(plb, 1, 0) + l_tr_set(plb, 1, 1)))
            mf += dvdk_group(os_, 1)
        if i + 1 < n:
            nlb = blocks[i + 1][0]
            if i >= 1:
                mf.append(('L', [l_rows(nlb, kk, t) for kk in range(KK) for t in (0, 1)] +
                           [l_init(os_, nlb, a, w) for w in (1, 0) for a in range(4)]))
            mf += sdp_products(os_)
        # block i's m = 0 transposed fragments, for its dK/dV in the next round
        mf.append(('L', l_tr_set(lb, 0, 1) + l_tr_set(lb, 0, 0)))
        n_m = sum(1 for x in mf if not isinstance(x, tuple))
        per = g.even(len(sm), max(n_m, 1))
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
    # the last block's dK/dV
    llb = blocks[-1][0]
    ls = (n - 1) % 2
    ops += dvdk_group(ls, 0) + l_tr_set(llb, 1, 0) + l_tr_set(llb, 1, 1) + dvdk_group(ls, 1)
    return g.hoist_lds(ops)


VARIANTS = {
    'FULL': ([(b, False) for b in range(4)], 'all four 32-row blocks below the diagonal'),
}
for _w in range(4):
    VARIANTS[f'DIAG{_w}'] = ([(_w, True)] + [(b, False) for b in range(_w + 1, 4)],
                             f'blocks {_w}..3 of the diagonal stage for wave {_w}')

DEFAULT_OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'dkdv128_item.inc')


def streams():
    out = []
    for name, (blocks, desc) in VARIANTS.items():
        e = g.Emitter()
        e.lines.append('s_waitcnt lgkmcnt(0)')
        for op in schedule_stage(blocks):
            e.emit(op)
        e.finish()
        out.append((name, desc, e))
    return out


def render(verbose=False):
    """The text of dkdv128_item.inc."""
    text = ['// Generated by gen_dkdv128_asm.py (do not edit): the instruction streams of one\n'
            '// 128-row stage of the D = 128 dK/dV pass for one wave, one per causal-mask case,\n'
            '// selected by the mode operand (0: FULL, 1 + w: DIAG<w>).\n']
    lines = ['s_nop 1']
    st = streams()
    for i, (name, _, _) in enumerate(st[1:], 1):
        lines += [f's_cmp_eq_u32 %{OP_MODE}, {i}', f's_cbranch_scc1 .Ldk128_{name}_%=']
    for i, (name, desc, e) in enumerate(st):
        n_mfma = sum(1 for l in e.lines if l.startswith('v_mfma'))
        n_lds = sum(1 for l in e.lines if l.startswith('ds_'))
        n_valu = sum(1 for l in e.lines if l.startswith('v_') and not l.startswith('v_mfma'))
        text.append(f'// {name}: {desc}; {n_mfma} MFMA, {n_lds} LDS reads, {n_valu} VALU, '
                    f'{e.n_waits} lgkmcnt waits, {e.n_nops} nop wait states.\n')
        if verbose:
            print(f'{name}: {n_mfma} MFMA, {n_lds} LDS, {n_valu} VALU, {e.n_waits} waits, {e.n_nops} nops')
        if i > 0:
            lines.append(f'.Ldk128_{name}_%=:')
        lines += e.lines
        if i < len(st) - 1:
            lines.append('s_branch .Ldk128_end_%=')
    lines.append('.Ldk128_end_%=:')
    body = ''.join(f'  "{l}\\n"\n' for l in lines)
    text.append('#define TTFA_DKDV128_STAGE_ASM \\\n' + body.rstrip('\n').replace('\n', ' \\\n') + '\n')
    clob = ', '.join(f'"v{i}"' for i in range(N_VTEMP))
    text.append(f'\n#define TTFA_DKDV128_ITEM_CLOBBERS {clob}, "vcc", "scc"\n')
    return ''.join(text)


def main():
    out = sys.argv[1] if len(sys.argv) > 1 else DEFAULT_OUT
    with open(out, 'w') as f:
        f.write(render(verbose=True))
    print(f'wrote {out}')


if __name__ == '__main__':
    main()
