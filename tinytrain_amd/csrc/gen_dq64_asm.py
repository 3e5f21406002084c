#!/usr/bin/env python3
"""Writes dq64_stage.inc: the instruction stream of one 128-key stage of the D = 64 dQ pass
(fa_bwd_dq64.hip) for one wave (32 query rows), as the text of one inline-asm statement.

Per 32-key block the wave issues 12 MFMAs (S^T = K Q^T and dP^T = V dO^T, 4 k-steps each,
then dQ^T += K^T dS^T, 2 row groups x 2 column blocks), 16 LDS operand reads and ~72 VALU
operations.  As in the dK/dV pass (gen_dkdv64_asm.py, whose emitter and LDS placement this
reuses), the stage's four blocks form a software pipeline: round i runs block i's
exponentials on the VALU under block i-1's dQ products and block i+1's S^T/dP^T products,
in two alternating register sets, with every LDS read issued ahead of its use and the
waits and hazard padding inserted by the emitter.

Each lane owns one query row (lq) and 16 of a block's 32 keys (rows 8a+4lg+e of the S^T
result), so LSE and Delta are per-lane scalars: P^T = exp2(S^T * scale*log2e - LSE*log2e)
is one FMA and one exp per score, the dP^T accumulator starts at -Delta (16 moves), and
dS^T = P^T (dP^T - Delta) one multiply.

Register map (fixed; the statement clobbers v[0:111]):
  v[0:15] S^T of register set 0 (then P^T), v[16:31] its dP^T (then dS^T, packed to bf16
  in place: keys 8m..8m+7 of the block into registers 8m..8m+3), v[32:63] set 1;
  v[64:79] K row fragments (A operands of S^T, k-step kk at v[64+4kk]), v[80:95] V row
  fragments, v[96:111] K^T fragments (16-key row group m at v[96+8m], column block db
  at +4db).
Operands: %0, %1 the dQ^T accumulators (AGPR, db = 0, 1), %2..%5 the Q fragments and
%6..%9 the dO fragments (AGPR B operands, k-step kk), %10..%13 the LDS byte addresses of
the K row reads per k-step (V rows: + V_OFF), %14..%17 those of the K^T reads
([db][h]), %18 the SGPR scale*log2(e), %19 -LSE*log2(e), %20 -Delta, %21 the mask bound
(a key is masked when its offset in the stage minus 4lg exceeds it), %22 the SGPR mode.

Variants (mode): FULL (0), the stage that holds wave w's diagonal, DIAG<w> (1 + w: blocks
0..w, block w masked), and RAGGED (5: every block masked by the bound, for the stage that
crosses T; keys at or past T must not count, their P would be exp2(-LSE) times zero K rows
but could overflow for extreme LSE).

usage: python gen_dq64_asm.py [out.inc]
"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import gen_dkdv64_asm as g  # noqa: E402  (emitter, LDS placement, helpers)

Op, vr, vt = g.Op, g.vr, g.vt

STAGE_KEYS = 128
V_OFF = STAGE_KEYS * 128    # V tile after the K tile in a stage (bytes)

S = [0, 32]
P = [16, 48]
KR, VR, KT = 64, 80, 96   # K^T fragments of row group m at v[96+8m : 103+8m]
N_VTEMP = 112

OP_DQ = [0, 1]
OP_QF = [2, 3, 4, 5]
OP_DF = [6, 7, 8, 9]
OP_AR = [10, 11, 12, 13]
OP_AT = [[14, 15], [16, 17]]
OP_SCALE = 18
OP_NLSE = 19
OP_NDELTA = 20
OP_DM = 21
OP_MODE = 22


def l_krow(lb, kk):
    dst = KR + 4 * kk
    return Op(f'ds_read_b128 {vt(dst, 4)}, %{OP_AR[kk]} offset:{4096 * lb}', 'lds', writes=vr(dst, 4))


def l_vrow(lb, kk):
    dst = VR + 4 * kk
    return Op(f'ds_read_b128 {vt(dst, 4)}, %{OP_AR[kk]} offset:{V_OFF + 4096 * lb}', 'lds', writes=vr(dst, 4))


def l_kt(lb, m, db, h):
    """Half h of the K^T fragment (keys 32lb+16m.., d columns 32db..)."""
    dst = KT + 8 * m + 4 * db + 2 * h
    off = (32 * lb + 16 * m) * 128
    return Op(f'ds_read_b64_tr_b16 {vt(dst, 2)}, %{OP_AT[db][h]} offset:{off}', 'lds', writes=vr(dst, 2))


def l_kt_set(lb, m):
    return [l_kt(lb, m, db, h) for db in range(2) for h in range(2)]


def init_dp(rs):
    return [Op(f'v_mov_b32 v{P[rs] + r}, %{OP_NDELTA}', 'valu', writes=[f'v{P[rs] + r}']) for r in range(16)]


def m_s(rs, kk):
    src_c = '0' if kk == 0 else vt(S[rs], 16)
    reads = vr(KR + 4 * kk, 4) + ([] if kk == 0 else vr(S[rs], 16))
    return Op(f'v_mfma_f32_32x32x16_bf16 {vt(S[rs], 16)}, {vt(KR + 4 * kk, 4)}, %{OP_QF[kk]}, {src_c}',
              'mfma', reads=reads, writes=vr(S[rs], 16))


def m_p(rs, kk):
    return Op(f'v_mfma_f32_32x32x16_bf16 {vt(P[rs], 16)}, {vt(VR + 4 * kk, 4)}, %{OP_DF[kk]}, {vt(P[rs], 16)}',
              'mfma', reads=vr(P[rs], 16) + vr(VR + 4 * kk, 4), writes=vr(P[rs], 16))


def m_dq(rs, m, db):
    acc = f'%{OP_DQ[db]}'
    kt = KT + 8 * m + 4 * db
    return Op(f'v_mfma_f32_32x32x16_bf16 {acc}, {vt(kt, 4)}, {vt(P[rs] + 8 * m, 4)}, {acc}',
              'mfma', reads=vr(kt, 4) + vr(P[rs] + 8 * m, 4) + [acc], writes=[acc])


def softmax(rs, lb, masked):
    """P^T = exp2(S^T * scale*log2e - LSE*log2e), masked to 0 where the key's offset in
    the stage minus 4lg exceeds the bound; dS^T = P^T (dP^T - Delta) in place; dS^T
    packed to bf16 in place."""
    ops = []
    s, p = S[rs], P[rs]
    for m in range(2):
        for r0 in range(8 * m, 8 * m + 8, 2):
            for r in (r0, r0 + 1):
                ops.append(Op(f'v_fma_f32 v{s + r}, v{s + r}, %{OP_SCALE}, %{OP_NLSE}', 'valu',
                              reads=[f'v{s + r}'], writes=[f'v{s + r}']))
            for r in (r0, r0 + 1):
                ops.append(Op(f'v_exp_f32 v{s + r}, v{s + r}', 'trans', reads=[f'v{s + r}'], writes=[f'v{s + r}']))
            if masked:  # P = 0 for masked keys (exp2(-inf) = +0 in the unscheduled code)
                for r in (r0, r0 + 1):
                    c = 32 * lb + 8 * (r >> 2) + (r & 3)
                    ops.append(Op(f'v_cmp_gt_i32 vcc, {c}, %{OP_DM}', 'valu', writes=['vcc']))
                    ops.append(Op(f'v_cndmask_b32_e64 v{s + r}, v{s + r}, 0, vcc', 'valu',
                                  reads=[f'v{s + r}', 'vcc'], writes=[f'v{s + r}']))
            for r in (r0, r0 + 1):
                ops.append(Op(f'v_mul_f32 v{p + r}, v{s + r}, v{p + r}', 'valu',
                              reads=[f'v{s + r}', f'v{p + r}'], writes=[f'v{p + r}']))
        for j in range(4):
            a, b = p + 8 * m + 2 * j, p + 8 * m + 2 * j + 1
            ops.append(Op(f'v_cvt_pk_bf16_f32 v{p + 8 * m + j}, v{a}, v{b}', 'valu',
                          reads=[f'v{a}', f'v{b}'], writes=[f'v{p + 8 * m + j}']))
    return ops


def dq_products(rs):
    """The dQ products of a block in register set rs: row groups m = 0, 1, column blocks."""
    return [m_dq(rs, m, db) for m in range(2) for db in range(2)]


def sd_products(rs):
    out = []
    for kk in range(4):
        out += [m_s(rs, kk), m_p(rs, kk)]
    return out


def schedule_stage(blocks):
    """blocks: list of (lds block, masked), block i in register set i % 2."""
    n = len(blocks)
    ops = []
    lb0 = blocks[0][0]
    ops += [x for kk in range(4) for x in (l_krow(lb0, kk), l_vrow(lb0, kk))]
    ops += init_dp(0)
    ops += sd_products(0)
    if n > 1:
        lb1 = blocks[1][0]
        ops += [x for kk in range(4) for x in (l_krow(lb1, kk), l_vrow(lb1, kk))]
    for i in range(n):
        lb, masked = blocks[i]
        rs, os_ = i % 2, 1 - i % 2
        sm = softmax(rs, lb, masked)
        mf = []
        if i >= 1:
            mf += dq_products(os_)
        if i + 1 < n:
            nlb = blocks[i + 1][0]
            if i >= 1:
                mf.append(('L', [x for kk in range(4) for x in (l_krow(nlb, kk), l_vrow(nlb, kk))]))
            mf.append(('V', init_dp(os_)))
            mf += sd_products(os_)
        # block i's K^T fragments, for its dQ products in the next round
        mf.append(('L', l_kt_set(lb, 0) + l_kt_set(lb, 1)))
        n_m = sum(1 for x in mf if isinstance(x, Op) and x.kind == 'mfma')
        per = g.even(len(sm), max(n_m, 1))
        k = j = 0
        for x in mf:
            if isinstance(x, tuple):
                ops += x[1]
                continue
            ops.append(x)
            if x.kind != 'mfma':
                continue
            ops += sm[k:k + per[j]]
            k += per[j]
            j += 1
        ops += sm[k:]
    ops += dq_products((n - 1) % 2)
    return g.hoist_lds(ops)


VARIANTS = {'FULL': ([(b, False) for b in range(4)], 'every key of the stage precedes every row of the wave')}
for _w in range(4):
    VARIANTS[f'DIAG{_w}'] = ([(b, False) for b in range(_w)] + [(_w, True)],
                             f'the stage holding wave {_w}\'s diagonal: blocks 0..{_w}, block {_w} masked')
VARIANTS['RAGGED'] = ([(b, True) for b in range(4)], 'the stage that crosses T: every block masked')

DEFAULT_OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'dq64_stage.inc')


def render(verbose=False):
    names = list(VARIANTS)
    text = ['// Generated by gen_dq64_asm.py (do not edit): the instruction streams of one 128-key\n'
            '// stage of the D = 64 dQ pass for one wave, one per mask case, selected by the mode\n'
            '// operand (0: FULL, 1 + w: DIAG<w>, 5: RAGGED).\n']
    lines = ['s_nop 1']
    for i, name in enumerate(names[1:], 1):
        lines += [f's_cmp_eq_u32 %{OP_MODE}, {i}', f's_cbranch_scc1 .Ldq_{name}_%=']
    for i, name in enumerate(names):
        blocks, desc = VARIANTS[name]
        e = g.Emitter()
        e.lines.append('s_waitcnt lgkmcnt(0)')
        for op in schedule_stage(blocks):
            e.emit(op)
        e.finish()
        n_mfma = sum(1 for l in e.lines if l.startswith('v_mfma'))
        n_lds = sum(1 for l in e.lines if l.startswith('ds_'))
        n_valu = sum(1 for l in e.lines if l.startswith('v_') and not l.startswith('v_mfma'))
        text.append(f'// {name}: {desc}; {n_mfma} MFMA, {n_lds} LDS reads, {n_valu} VALU, '
                    f'{e.n_waits} lgkmcnt waits, {e.n_nops} nop wait states.\n')
        if verbose:
            print(f'{name}: {n_mfma} MFMA, {n_lds} LDS, {n_valu} VALU, {e.n_waits} waits, {e.n_nops} nops')
        if i > 0:
            lines.append(f'.Ldq_{name}_%=:')
        lines += e.lines
        if i < len(names) - 1:
            lines.append('s_branch .Ldq_end_%=')
    lines.append('.Ldq_end_%=:')
    body = ''.join(f'  "{l}\\n"\n' for l in lines)
    text.append('#define TTFA_DQ64_STAGE_ASM \\\n' + body.rstrip('\n').replace('\n', ' \\\n') + '\n')
    clob = ', '.join(f'"v{i}"' for i in range(N_VTEMP))
    text.append(f'\n#define TTFA_DQ64_STAGE_CLOBBERS {clob}, "vcc", "scc"\n')
    return ''.join(text)


def main():
    out = sys.argv[1] if len(sys.argv) > 1 else DEFAULT_OUT
    with open(out, 'w') as f:
        f.write(render(verbose=True))
    print(f'wrote {out}')


if __name__ == '__main__':
    main()
