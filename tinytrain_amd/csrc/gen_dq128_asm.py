#!/usr/bin/env python3
"""Writes dq128_stage.inc: the instruction stream of one 128-key stage of the D = 128 dQ
pass (fa_bwd_dq128.hip) for one wave, as the text of one inline-asm statement.

The wave owns 64 query rows, two 32-row groups qg, whose Q and dO fragments (the B
operands of S^T = K Q^T and dP^T = V dO^T) and dQ^T accumulators stay in AGPRs.  Each K/V
row fragment and each K^T fragment read from LDS feeds one product per row group, so a
product costs half the LDS bytes of a 32-row wave (LDS delivery, not the matrix cores,
bounds the 32-row form of this pass).  The work items of a stage are (32-key block b, row
group qg), in the order (b0,q0), (b0,q1), (b1,q0), ...; an item is 16 S^T/dP^T products,
56 VALU operations (P^T = exp2(S^T * scale*log2e - LSE*log2e), dS^T = P^T (dP^T -
Delta), packed to bf16; 32 more where masked) and 8 dQ^T products (dQ^T += K^T dS^T, 2 key row groups m x 4
column blocks db).  As in the dK/dV passes (gen_dkdv64_asm.py, whose emitter and LDS
placement this reuses), the items form a software pipeline: round i runs item i's VALU
work under item i-1's dQ^T products and item i+1's S^T/dP^T products, in two alternating
register sets.

Register map (fixed; the statement clobbers v[0:175]):
  v[0:15] S^T of register set 0, v[16:31] its dP^T (then dS^T, packed to bf16 in place:
  keys 8m..8m+7 of the block into registers 8m..8m+3), v[32:63] set 1; v[64+4kk] K row
  fragments of the current block, v[96+4kk] V row fragments, v[128+16m+4db] K^T
  fragments (key row group m, column block db); v[160+kk] the LDS addresses of the row
  reads of k-step kk, v[168+2db+h] those of the transposed reads (column block db, 8-row
  half h).
AGPR state (fixed registers, written by TTFA_DQ128_INIT_ASM, read back by
TTFA_DQ128_READ_ASM, and held between the statements because every statement of the pass
declares all AGPRs clobbered, so the compiler keeps nothing there): a[64qg+16db : +15]
the dQ^T accumulators (row group qg, column block db), a[128+32qg+4kk : +3] the Q
fragments, a[192+32qg+4kk : +3] the dO fragments.
Operands: %0 the lane's LDS byte address of the k-step 0 row read of key block 0 (K
tile; the V tile at +32768), %1 that of its transposed read for column block 0, half 0;
%2 the SGPR scale*log2(e); %3, %4 -LSE*log2(e) of the lane's row in each row group;
%5, %6 -Delta; %7, %8 the mask bounds (a key is masked when its offset in the stage minus
4lg exceeds the bound); %9 the SGPR mode (0: FULL, 1: MASKED); %10, %11 16-register
blocks holding -Delta in every register (the C operand of each row group's first dP^T
product, so no item spends moves on its start value).
The tiles use swz_rows128 (row bits 0-3 XOR all four chunk bits), so with the stage
base 256-byte aligned the row read of k-step kk is at %40 ^ 32kk and the transposed read
of (db, h) at (%41 ^ (64db + 32h)) + 2048h; the key blocks (+8192 bytes) and key row
groups (+4096) are immediate offsets.

Variants (mode): FULL, the stage lies below both row groups (every key visible), and
MASKED, every item masked by its row group's bound (the diagonal stages and the stage that
crosses T: keys at or past T must not count, their P would be exp2(-LSE) times zero K
rows but could overflow for extreme LSE).  A wave whose rows see no key of a stage skips
the statement.

usage: python gen_dq128_asm.py [out.inc]
"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import gen_dkdv64_asm as g  # noqa: E402  (emitter, LDS placement, helpers)

Op, vr, vt = g.Op, g.vr, g.vt

KK = 8                      # k-steps of S^T and dP^T (D = 128)
DB = 4                      # column blocks of dQ^T
ROW_BYTES = 256
STAGE_KEYS = 128
V_OFF = STAGE_KEYS * ROW_BYTES   # V tile after the K tile in a stage (bytes)
BLOCK_BYTES = 32 * ROW_BYTES

S = [0, 32]
P = [16, 48]
KR, VR, KT = 64, 96, 128
AR, AT = 160, 168
N_VTEMP = 176

# The wave's AGPR state lives in fixed registers that only this file's statements touch
# (all 256 AGPRs: as asm operands the compiler either does not finish allocating them or
# copies them through spilled VGPRs every stage): dQ^T accumulators a[0:127], Q fragments
# a[128:191], dO fragments a[192:255].
A_DQ = [[f'a[{64 * qg + 16 * db}:{64 * qg + 16 * db + 15}]' for db in range(4)] for qg in range(2)]
A_QF = [[f'a[{128 + 32 * qg + 4 * kk}:{128 + 32 * qg + 4 * kk + 3}]' for kk in range(8)] for qg in range(2)]
A_DF = [[f'a[{192 + 32 * qg + 4 * kk}:{192 + 32 * qg + 4 * kk + 3}]' for kk in range(8)] for qg in range(2)]
OP_AR0 = 0
OP_AT0 = 1
OP_SCALE = 2
OP_NLSE = [3, 4]
OP_NDELTA = [5, 6]
OP_DM = [7, 8]
OP_MODE = 9
OP_NDB = [10, 11]  # 16-register blocks of -Delta (the dP^T chains' start), per row group


def addresses():
    """The 16 LDS addresses of the stage from the two base operands."""
    ops = [Op(f'v_mov_b32 v{AR}, %{OP_AR0}', 'valu', writes=[f'v{AR}'])]
    ops += [Op(f'v_xor_b32 v{AR + kk}, {32 * kk}, %{OP_AR0}', 'valu', writes=[f'v{AR + kk}'])
            for kk in range(1, KK)]
    ops += [Op(f'v_mov_b32 v{AT}, %{OP_AT0}', 'valu', writes=[f'v{AT}'])]
    ops += [Op(f'v_xor_b32 v{AT + i}, {32 * i}, %{OP_AT0}', 'valu', writes=[f'v{AT + i}'])
            for i in range(1, 2 * DB)]
    return ops


def l_krow(lb, kk):
    dst = KR + 4 * kk
    return Op(f'ds_read_b128 {vt(dst, 4)}, v{AR + kk} offset:{BLOCK_BYTES * lb}', 'lds',
              reads=[f'v{AR + kk}'], writes=vr(dst, 4))


def l_vrow(lb, kk):
    dst = VR + 4 * kk
    return Op(f'ds_read_b128 {vt(dst, 4)}, v{AR + kk} offset:{V_OFF + BLOCK_BYTES * lb}', 'lds',
              reads=[f'v{AR + kk}'], writes=vr(dst, 4))


def l_rows(lb):
    return [x for kk in range(KK) for x in (l_krow(lb, kk), l_vrow(lb, kk))]


def l_kt(lb, m, db, h):
    """Half h of the K^T fragment (keys 32lb+16m.., d columns 32db..)."""
    dst = KT + 16 * m + 4 * db + 2 * h
    off = (32 * lb + 16 * m) * ROW_BYTES + 2048 * h
    return Op(f'ds_read_b64_tr_b16 {vt(dst, 2)}, v{AT + 2 * db + h} offset:{off}', 'lds',
              reads=[f'v{AT + 2 * db + h}'], writes=vr(dst, 2))


def l_kt_all(lb):
    return [l_kt(lb, m, db, h) for m in range(2) for db in range(DB) for h in range(2)]


def m_s(rs, qg, kk):
    src_c = '0' if kk == 0 else vt(S[rs], 16)
    reads = vr(KR + 4 * kk, 4) + ([] if kk == 0 else vr(S[rs], 16))
    return Op(f'v_mfma_f32_32x32x16_bf16 {vt(S[rs], 16)}, {vt(KR + 4 * kk, 4)}, {A_QF[qg][kk]}, {src_c}',
              'mfma', reads=reads, writes=vr(S[rs], 16))


def m_p(rs, qg, kk):
    src_c = f'%{OP_NDB[qg]}' if kk == 0 else vt(P[rs], 16)
    reads = vr(VR + 4 * kk, 4) + ([src_c] if kk == 0 else vr(P[rs], 16))
    return Op(f'v_mfma_f32_32x32x16_bf16 {vt(P[rs], 16)}, {vt(VR + 4 * kk, 4)}, {A_DF[qg][kk]}, {src_c}',
              'mfma', reads=reads, writes=vr(P[rs], 16))


def m_dq(rs, qg, m, db):
    acc = A_DQ[qg][db]
    kt = KT + 16 * m + 4 * db
    return Op(f'v_mfma_f32_32x32x16_bf16 {acc}, {vt(kt, 4)}, {vt(P[rs] + 8 * m, 4)}, {acc}',
              'mfma', reads=vr(kt, 4) + vr(P[rs] + 8 * m, 4) + [acc], writes=[acc])


def softmax(rs, qg, lb, masked):
    """P^T = exp2(S^T * scale*log2e - LSE*log2e), masked to 0 where the key's offset in
    the stage minus 4lg exceeds the row group's bound; dS^T = P^T (dP^T - Delta) in place;
    dS^T packed to bf16 in place."""
    ops = []
    s, p = S[rs], P[rs]
    for m in range(2):
        for r0 in range(8 * m, 8 * m + 8, 2):
            for r in (r0, r0 + 1):
                ops.append(Op(f'v_fma_f32 v{s + r}, v{s + r}, %{OP_SCALE}, %{OP_NLSE[qg]}', 'valu',
                              reads=[f'v{s + r}'], writes=[f'v{s + r}']))
            for r in (r0, r0 + 1):
                ops.append(Op(f'v_exp_f32 v{s + r}, v{s + r}', 'trans', reads=[f'v{s + r}'], writes=[f'v{s + r}']))
            if masked:  # P = 0 for masked keys
                for r in (r0, r0 + 1):
                    c = 32 * lb + 8 * (r >> 2) + (r & 3)
                    ops.append(Op(f'v_cmp_gt_i32 vcc, {c}, %{OP_DM[qg]}', 'valu', writes=['vcc']))
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


def dq_products(rs, qg):
    return [m_dq(rs, qg, m, db) for m in range(2) for db in range(DB)]


def sd_products(rs, qg):
    out = []
    for kk in range(KK):
        out += [m_s(rs, qg, kk), m_p(rs, qg, kk)]
    return out


def schedule_stage(masked):
    """The 8 items (block b, row group qg) of a stage; item i in register set i % 2."""
    items = [(b, qg) for b in range(4) for qg in range(2)]
    n = len(items)
    ops = addresses()
    ops += l_rows(0)
    ops += sd_products(0, 0)
    for i in range(n):
        b, qg = items[i]
        rs, os_ = i % 2, 1 - i % 2
        sm = softmax(rs, qg, b, masked)
        mf = []
        if i >= 1:
            mf += dq_products(os_, items[i - 1][1])
        if i + 1 < n:
            nb, nqg = items[i + 1]
            if nqg == 0:  # a new key block: its K/V rows replace block b's
                mf.append(('L', l_rows(nb)))
            mf += sd_products(os_, nqg)
        if qg == 0:  # block b's K^T fragments, for the dQ^T products of rounds i+1, i+2
            mf.append(('L', l_kt_all(b)))
        n_m = sum(1 for x in mf if isinstance(x, Op) and x.kind == 'mfma')
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
    ops += dq_products((n - 1) % 2, items[-1][1])
    return g.hoist_lds(ops)


VARIANTS = {
    'FULL': (False, 'every key of the stage precedes both row groups of the wave'),
    'MASKED': (True, 'a diagonal stage or the stage that crosses T: every item masked'),
}

DEFAULT_OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'dq128_stage.inc')


def streams():
    out = []
    for name, (masked, desc) in VARIANTS.items():
        e = g.Emitter()
        e.lines.append('s_waitcnt lgkmcnt(0)')
        for op in schedule_stage(masked):
            e.emit(op)
        e.finish()
        out.append((name, desc, e))
    return out


def render(verbose=False):
    """The text of dq128_stage.inc."""
    text = ['// Generated by gen_dq128_asm.py (do not edit): the instruction streams of one\n'
            '// 128-key stage of the D = 128 dQ pass for one wave (64 query rows), one per mask\n'
            '// case, selected by the mode operand (0: FULL, 1: MASKED).\n']
    lines = ['s_nop 1']
    st = streams()
    for i, (name, _, _) in enumerate(st[1:], 1):
        lines += [f's_cmp_eq_u32 %{OP_MODE}, {i}', f's_cbranch_scc1 .Ldq128_{name}_%=']
    for i, (name, desc, e) in enumerate(st):
        n_mfma = sum(1 for l in e.lines if l.startswith('v_mfma'))
        n_lds = sum(1 for l in e.lines if l.startswith('ds_'))
        n_valu = sum(1 for l in e.lines if l.startswith('v_') and not l.startswith('v_mfma'))
        text.append(f'// {name}: {desc}; {n_mfma} MFMA, {n_lds} LDS reads, {n_valu} VALU, '
                    f'{e.n_waits} lgkmcnt waits, {e.n_nops} nop wait states.\n')
        if verbose:
            print(f'{name}: {n_mfma} MFMA, {n_lds} LDS, {n_valu} VALU, {e.n_waits} waits, {e.n_nops} nops')
        if i > 0:
            lines.append(f'.Ldq128_{name}_%=:')
        lines += e.lines
        if i < len(st) - 1:
            lines.append('s_branch .Ldq128_end_%=')
    lines.append('.Ldq128_end_%=:')
    body = ''.join(f'  "{l}\\n"\n' for l in lines)
    text.append('#define TTFA_DQ128_STAGE_ASM \\\n' + body.rstrip('\n').replace('\n', ' \\\n') + '\n')
    clob = ', '.join(f'"v{i}"' for i in range(N_VTEMP))
    aclob = ', '.join(f'"a{i}"' for i in range(256))
    text.append(f'\n#define TTFA_DQ128_AGPR_CLOBBERS {aclob}\n')
    text.append(f'\n#define TTFA_DQ128_STAGE_CLOBBERS {clob}, TTFA_DQ128_AGPR_CLOBBERS, "vcc", "scc"\n')
    # set-up: Q fragments (inputs v[0:63], fragment 8qg+kk at v[4(8qg+kk)]) and dO
    # fragments (v[64:127]) into their AGPRs, accumulators zeroed; 2 wait states before an
    # MFMA reads an AGPR a VALU wrote
    init = [f'v_accvgpr_write_b32 a{128 + i}, v{i}' for i in range(128)]
    init += [f'v_accvgpr_write_b32 a{i}, 0' for i in range(128)]
    init += ['s_nop 1']
    body = ''.join(f'  "{l}\\n"\n' for l in init)
    text.append('\n// Moves the wave\'s Q and dO fragments into their AGPRs and zeroes the accumulators.\n')
    text.append('#define TTFA_DQ128_INIT_ASM \\\n' + body.rstrip('\n').replace('\n', ' \\\n') + '\n')
    # read-back: accumulator (qg, db) into v[16(4qg+db) : +15] (the stage statements end
    # with the wait states a VALU read of a product needs)
    rd = [f'v_accvgpr_read_b32 v{i}, a{i}' for i in range(128)]
    body = ''.join(f'  "{l}\\n"\n' for l in rd)
    text.append('\n// Reads the dQ^T accumulators back into v[0:127].\n')
    text.append('#define TTFA_DQ128_READ_ASM \\\n' + body.rstrip('\n').replace('\n', ' \\\n') + '\n')
    return ''.join(text)


def main():
    out = sys.argv[1] if len(sys.argv) > 1 else DEFAULT_OUT
    with open(out, 'w') as f:
        f.write(render(verbose=True))
    print(f'wrote {out}')


if __name__ == '__main__':
    main()
