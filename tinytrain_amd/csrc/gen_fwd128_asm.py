#!/usr/bin/env python3
"""Writes fwd128_stage.inc: the instruction stream of one 128-key stage of the D = 128
forward over 256-row tiles (fa_fwd128.hip) for one wave, as the text of one inline-asm
statement.

The wave owns 64 query rows, two 32-row groups qg, whose Q fragments (the B operands of
S^T = K Q^T) and O^T accumulators stay in fixed AGPRs.  Each K row fragment and V^T
fragment read from LDS feeds one product per row group: half the LDS bytes per product of
a 32-row wave.  The work items of a stage are (32-key block b, row group qg), in the order
(b0,q0), (b0,q1), (b1,q0), ...; an item is 8 S^T products, the online softmax on the
VALU (row max over the item's 32 keys as a maximum3 tree, a lazy rescale of O and l
when the max grows by more than 2^8, P^T = exp2(S^T * scale*log2e - m), the row sum in
four partial sums, P^T packed to bf16) and 8
PV products (O^T += V^T P^T, 2 key row groups m x 4 column blocks db).  As in the
backward streams (gen_dkdv64_asm.py, whose emitter and LDS placement this reuses), the
items form a software pipeline: round i runs item i's VALU work under item i-1's PV
products and item i+1's S^T products, in two alternating register sets.

Register map (fixed; the statement clobbers v[0:121]):
  v[0:15] S^T of register set 0 (then P^T, packed to bf16 in place: keys 8m..8m+7 of the
  block into registers 8m..8m+3), v[16:31] set 1; v[32+4kk] K row fragments of the
  current block; v[64+16m+4db] V^T fragments (key row group m, column block db);
  v[96+kk] the LDS addresses of the K row reads of k-step kk, v[104+2db+h] those of the
  V^T reads (column block db, 8-row half h); v[112:121] temporaries (the max tree's
  partials, -inf, the rescale factor and new max, the rescale's O copies, the row sum's
  four partial sums).
AGPR state (fixed registers, written by TTFA_FWD128_INIT_ASM, read back by
TTFA_FWD128_READ_ASM, held between the statements because every statement of the pass
declares all AGPRs clobbered): a[64qg+16db : +15] the O^T accumulators (row group qg,
column block db), a[128+32qg+4kk : +3] the Q fragments.
Operands: %0, %1 the running row max of the lane's row in each row group (scale*log2e
units), %2, %3 its share of the running row sum, %4 the lane's LDS byte address of the
k-step 0 K row read of key block 0, %5 that of its V^T read for column block 0, half 0
(the V tile at +32768), %6 the SGPR scale*log2(e), %7, %8 the mask bounds (a key is
masked when its offset in the stage minus 4lg exceeds the bound), %9 the SGPR mode
(0: FULL, 1: MASKED).  The tiles use swz_rows128, so with the stage base 256-byte aligned
the K row read of k-step kk is at %4 ^ 32kk and the V^T read of (db, h) at
(%5 ^ (64db + 32h)) + 2048h; key blocks (+8192 bytes) and key row groups (+4096) are
immediate offsets.

Variants (mode): FULL, every key of the stage visible to both row groups, and MASKED,
every item masked by its row group's bound before the row max (the diagonal stages and
the stage that crosses T).  A wave whose rows see no key of a stage skips the statement.
The first item a row group sees always holds a visible key (key 0), so the running max
is finite from then on and masked scores give P = exp2(-inf) = 0.

usage: python gen_fwd128_asm.py [out.inc]
"""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import gen_dkdv64_asm as g  # noqa: E402  (emitter, LDS placement, helpers)

Op, vr, vt = g.Op, g.vr, g.vt

KK = 8
DB = 4
ROW_BYTES = 256
STAGE_KEYS = 128
V_OFF = STAGE_KEYS * ROW_BYTES
BLOCK_BYTES = 32 * ROW_BYTES
RESCALE_SLACK = 8.0

S = [0, 16]
KR, VT_, AR, AT = 32, 64, 96, 104
T_MX, T_SW, T_NINF, T_ALPHA, T_MN, T_AC = 112, 113, 114, 115, 116, 117  # temporaries (117-121)
N_VTEMP = 122

A_O = [[f'a[{64 * qg + 16 * db}:{64 * qg + 16 * db + 15}]' for db in range(DB)] for qg in range(2)]
A_QF = [[f'a[{128 + 32 * qg + 4 * kk}:{128 + 32 * qg + 4 * kk + 3}]' for kk in range(KK)] for qg in range(2)]
OP_M = [0, 1]
OP_L = [2, 3]
OP_AR0 = 4
OP_AT0 = 5
OP_SCALE = 6
OP_DM = [7, 8]
OP_MODE = 9


def o_regs(qg):
    return [f'a{64 * qg + i}' for i in range(64)]


def addresses():
    ops = [Op(f'v_mov_b32 v{AR}, %{OP_AR0}', 'valu', writes=[f'v{AR}'])]
    ops += [Op(f'v_xor_b32 v{AR + kk}, {32 * kk}, %{OP_AR0}', 'valu', writes=[f'v{AR + kk}'])
            for kk in range(1, KK)]
    ops += [Op(f'v_mov_b32 v{AT}, %{OP_AT0}', 'valu', writes=[f'v{AT}'])]
    ops += [Op(f'v_xor_b32 v{AT + i}, {32 * i}, %{OP_AT0}', 'valu', writes=[f'v{AT + i}'])
            for i in range(1, 2 * DB)]
    ops += [Op(f'v_mov_b32 v{T_NINF}, 0xff800000', 'valu', writes=[f'v{T_NINF}'])]
    return ops


def l_krow(lb, kk):
    dst = KR + 4 * kk
    return Op(f'ds_read_b128 {vt(dst, 4)}, v{AR + kk} offset:{BLOCK_BYTES * lb}', 'lds',
              reads=[f'v{AR + kk}'], writes=vr(dst, 4))


def l_rows(lb):
    return [l_krow(lb, kk) for kk in range(KK)]


def l_vt(lb, m, db, h):
    """Half h of the V^T fragment (keys 32lb+16m.., d columns 32db..)."""
    dst = VT_ + 16 * m + 4 * db + 2 * h
    off = V_OFF + (32 * lb + 16 * m) * ROW_BYTES + 2048 * h
    return Op(f'ds_read_b64_tr_b16 {vt(dst, 2)}, v{AT + 2 * db + h} offset:{off}', 'lds',
              reads=[f'v{AT + 2 * db + h}'], writes=vr(dst, 2))


def l_vt_all(lb):
    return [l_vt(lb, m, db, h) for m in range(2) for db in range(DB) for h in range(2)]


def m_s(rs, qg, kk):
    src_c = '0' if kk == 0 else vt(S[rs], 16)
    reads = vr(KR + 4 * kk, 4) + ([] if kk == 0 else vr(S[rs], 16))
    return Op(f'v_mfma_f32_32x32x16_bf16 {vt(S[rs], 16)}, {vt(KR + 4 * kk, 4)}, {A_QF[qg][kk]}, {src_c}',
              'mfma', reads=reads, writes=vr(S[rs], 16))


def m_pv(rs, qg, m, db):
    acc = A_O[qg][db]
    regs = [f'a{64 * qg + 16 * db + i}' for i in range(16)]
    vtr = VT_ + 16 * m + 4 * db
    return Op(f'v_mfma_f32_32x32x16_bf16 {acc}, {vt(vtr, 4)}, {vt(S[rs] + 8 * m, 4)}, {acc}',
              'mfma', reads=vr(vtr, 4) + vr(S[rs] + 8 * m, 4) + regs, writes=regs)


def rescale(qg, label):
    """The lazy rescale as one indivisible op (no LDS read may be placed inside it): when
    any lane's new max exceeds its running max by more than the slack, every lane takes
    m' = max(m, mx), scales O and l by exp2(m - m') and keeps m'."""
    m, l = f'%{OP_M[qg]}', f'%{OP_L[qg]}'
    lines = [f'v_add_f32 v{T_ALPHA}, {RESCALE_SLACK}, {m}',
             f'v_cmp_gt_f32 vcc, v{T_MX}, v{T_ALPHA}',
             f's_cbranch_vccz {label}',
             f'v_maximum3_f32 v{T_MN}, {m}, v{T_MX}, v{T_MX}',
             f'v_sub_f32 v{T_ALPHA}, {m}, v{T_MN}',
             f'v_exp_f32 v{T_ALPHA}, v{T_ALPHA}',
             f'v_mov_b32 {m}, v{T_MN}',
             's_nop 0',
             f'v_mul_f32 {l}, {l}, v{T_ALPHA}']
    # O *= alpha through VGPRs, four registers at a time
    for i in range(0, 64, 4):
        regs = [64 * qg + i + k for k in range(4)]
        lines += [f'v_accvgpr_read_b32 v{T_AC + k}, a{r}' for k, r in enumerate(regs)]
        lines += [f'v_mul_f32 v{T_AC + k}, v{T_AC + k}, v{T_ALPHA}' for k in range(4)]
        lines += [f'v_accvgpr_write_b32 a{r}, v{T_AC + k}' for k, r in enumerate(regs)]
    lines.append(f'{label}:')
    reads = [f'v{T_MX}', m, l] + o_regs(qg)
    writes = [m, l, 'vcc', f'v{T_ALPHA}', f'v{T_MN}'] + [f'v{T_AC + k}' for k in range(4)] + o_regs(qg)
    return Op('\n'.join(lines), 'valu', reads=reads, writes=writes)


def softmax(rs, qg, lb, masked, label):
    ops = []
    s = S[rs]
    if masked:  # masked scores become -inf before the row max
        for r in range(16):
            c = 32 * lb + 8 * (r >> 2) + (r & 3)
            ops.append(Op(f'v_cmp_gt_i32 vcc, {c}, %{OP_DM[qg]}', 'valu', writes=['vcc']))
            ops.append(Op(f'v_cndmask_b32_e64 v{s + r}, v{s + r}, v{T_NINF}, vcc', 'valu',
                          reads=[f'v{s + r}', f'v{T_NINF}', 'vcc'], writes=[f'v{s + r}']))
    # row max: a maximum3 tree (depth 3) over the lane's 16 scores, then across the two
    # lane halves; one wave per SIMD issues nothing else while a dependent chain waits
    part = [T_MX, T_SW, T_AC, T_AC + 1, T_AC + 2]
    for k, d in enumerate(part):
        src = [s + 3 * k, s + 3 * k + 1, s + 3 * k + 2]
        ops.append(Op(f'v_maximum3_f32 v{d}, v{src[0]}, v{src[1]}, v{src[2]}', 'valu',
                      reads=[f'v{x}' for x in src], writes=[f'v{d}']))
    ops.append(Op(f'v_maximum3_f32 v{T_MX}, v{T_MX}, v{T_SW}, v{T_AC}', 'valu',
                  reads=[f'v{T_MX}', f'v{T_SW}', f'v{T_AC}'], writes=[f'v{T_MX}']))
    ops.append(Op(f'v_maximum3_f32 v{T_SW}, v{T_AC + 1}, v{T_AC + 2}, v{s + 15}', 'valu',
                  reads=[f'v{T_AC + 1}', f'v{T_AC + 2}', f'v{s + 15}'], writes=[f'v{T_SW}']))
    ops.append(Op(f'v_maximum3_f32 v{T_MX}, v{T_MX}, v{T_SW}, v{T_SW}', 'valu',
                  reads=[f'v{T_MX}', f'v{T_SW}'], writes=[f'v{T_MX}']))
    ops.append(Op(f'v_mov_b32 v{T_SW}, v{T_MX}', 'valu', reads=[f'v{T_MX}'], writes=[f'v{T_SW}']))
    ops.append(Op(f's_nop 1\nv_permlane32_swap_b32 v{T_MX}, v{T_SW}', 'valu',
                  reads=[f'v{T_MX}', f'v{T_SW}'], writes=[f'v{T_MX}', f'v{T_SW}']))
    ops.append(Op(f'v_maximum3_f32 v{T_MX}, v{T_MX}, v{T_SW}, v{T_SW}', 'valu',
                  reads=[f'v{T_MX}', f'v{T_SW}'], writes=[f'v{T_MX}']))
    ops.append(Op(f'v_mul_f32 v{T_MX}, %{OP_SCALE}, v{T_MX}', 'valu', reads=[f'v{T_MX}'], writes=[f'v{T_MX}']))
    ops.append(rescale(qg, label))
    # P^T = exp2(S^T * scale*log2e - m), the row sum, P^T packed to bf16 in place
    m, l = f'%{OP_M[qg]}', f'%{OP_L[qg]}'
    for r0 in range(0, 16, 2):
        for r in (r0, r0 + 1):
            ops.append(Op(f'v_fma_f32 v{s + r}, v{s + r}, %{OP_SCALE}, -{m}', 'valu',
                          reads=[f'v{s + r}', m], writes=[f'v{s + r}']))
        for r in (r0, r0 + 1):
            ops.append(Op(f'v_exp_f32 v{s + r}, v{s + r}', 'trans', reads=[f'v{s + r}'], writes=[f'v{s + r}']))
    # the row sum in four partial sums (depth 5 instead of a 16-deep chain)
    acc = [T_AC + k for k in range(4)]
    for k in range(4):
        ops.append(Op(f'v_add_f32 v{acc[k]}, v{s + 2 * k}, v{s + 2 * k + 1}', 'valu',
                      reads=[f'v{s + 2 * k}', f'v{s + 2 * k + 1}'], writes=[f'v{acc[k]}']))
    for k in range(8, 16):
        a = acc[k % 4]
        ops.append(Op(f'v_add_f32 v{a}, v{a}, v{s + k}', 'valu', reads=[f'v{a}', f'v{s + k}'], writes=[f'v{a}']))
    ops.append(Op(f'v_add_f32 v{acc[0]}, v{acc[0]}, v{acc[1]}', 'valu', reads=[f'v{acc[0]}', f'v{acc[1]}'], writes=[f'v{acc[0]}']))
    ops.append(Op(f'v_add_f32 v{acc[2]}, v{acc[2]}, v{acc[3]}', 'valu', reads=[f'v{acc[2]}', f'v{acc[3]}'], writes=[f'v{acc[2]}']))
    ops.append(Op(f'v_add_f32 v{acc[0]}, v{acc[0]}, v{acc[2]}', 'valu', reads=[f'v{acc[0]}', f'v{acc[2]}'], writes=[f'v{acc[0]}']))
    ops.append(Op(f'v_add_f32 {l}, {l}, v{acc[0]}', 'valu', reads=[l, f'v{acc[0]}'], writes=[l]))
    for mm in range(2):
        for j in range(4):
            a, b = s + 8 * mm + 2 * j, s + 8 * mm + 2 * j + 1
            ops.append(Op(f'v_cvt_pk_bf16_f32 v{s + 8 * mm + j}, v{a}, v{b}', 'valu',
                          reads=[f'v{a}', f'v{b}'], writes=[f'v{s + 8 * mm + j}']))
    return ops


def pv_products(rs, qg):
    return [m_pv(rs, qg, m, db) for m in range(2) for db in range(DB)]


def s_products(rs, qg):
    return [m_s(rs, qg, kk) for kk in range(KK)]


def schedule_stage(masked, name):
    items = [(b, qg) for b in range(4) for qg in range(2)]
    n = len(items)
    ops = addresses()
    ops += l_rows(0)
    ops += s_products(0, 0)
    for i in range(n):
        b, qg = items[i]
        rs, os_ = i % 2, 1 - i % 2
        sm = softmax(rs, qg, b, masked, f'.Lfr_{name}_{i}_%=')
        mf = []
        if i >= 1:
            mf += pv_products(os_, items[i - 1][1])
        if i + 1 < n:
            nb, nqg = items[i + 1]
            if nqg == 0:  # a new key block: its K rows replace block b's
                mf.append(('L', l_rows(nb)))
            mf += s_products(os_, nqg)
        if qg == 0:  # block b's V^T fragments, for the PV products of rounds i+1, i+2
            mf.append(('L', l_vt_all(b)))
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
    ops += pv_products((n - 1) % 2, items[-1][1])
    return g.hoist_lds(ops)


VARIANTS = {
    'FULL': (False, 'every key of the stage precedes both row groups of the wave'),
    'MASKED': (True, 'a diagonal stage or the stage that crosses T: every item masked'),
}

DEFAULT_OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'fwd128_stage.inc')


def streams():
    out = []
    for name, (masked, desc) in VARIANTS.items():
        e = g.Emitter()
        e.lines.append('s_waitcnt lgkmcnt(0)')
        for op in schedule_stage(masked, name):
            e.emit(op)
        e.finish()
        out.append((name, desc, e))
    return out


def render(verbose=False):
    """The text of fwd128_stage.inc."""
    text = ['// Generated by gen_fwd128_asm.py (do not edit): the instruction streams of one\n'
            '// 128-key stage of the D = 128 forward for one wave (64 query rows), one per mask\n'
            '// case, selected by the mode operand (0: FULL, 1: MASKED).\n']
    lines = ['s_nop 1']
    st = streams()
    for i, (name, _, _) in enumerate(st[1:], 1):
        lines += [f's_cmp_eq_u32 %{OP_MODE}, {i}', f's_cbranch_scc1 .Lfw_{name}_%=']
    for i, (name, desc, e) in enumerate(st):
        flat = [x for l in e.lines for x in l.split('\n')]
        n_mfma = sum(1 for l in flat if l.startswith('v_mfma'))
        n_lds = sum(1 for l in flat if l.startswith('ds_'))
        n_valu = sum(1 for l in flat if l.startswith('v_') and not l.startswith('v_mfma'))
        text.append(f'// {name}: {desc}; {n_mfma} MFMA, {n_lds} LDS reads, {n_valu} VALU (rescale '
                    f'paths included), {e.n_waits} lgkmcnt waits, {e.n_nops} nop wait states.\n')
        if verbose:
            print(f'{name}: {n_mfma} MFMA, {n_lds} LDS, {n_valu} VALU, {e.n_waits} waits, {e.n_nops} nops')
        if i > 0:
            lines.append(f'.Lfw_{name}_%=:')
        lines += flat
        if i < len(st) - 1:
            lines.append('s_branch .Lfw_end_%=')
    lines.append('.Lfw_end_%=:')
    body = ''.join(f'  "{l}\\n"\n' for l in lines)
    text.append('#define TTFA_FWD128_STAGE_ASM \\\n' + body.rstrip('\n').replace('\n', ' \\\n') + '\n')
    clob = ', '.join(f'"v{i}"' for i in range(N_VTEMP))
    aclob = ', '.join(f'"a{i}"' for i in range(256))
    text.append(f'\n#define TTFA_FWD128_AGPR_CLOBBERS {aclob}\n')
    text.append(f'\n#define TTFA_FWD128_STAGE_CLOBBERS {clob}, TTFA_FWD128_AGPR_CLOBBERS, "vcc", "scc"\n')
    # set-up: Q fragments (inputs v[0:63], fragment 8qg+kk at v[4(8qg+kk)]) into their AGPRs,
    # accumulators zeroed; 2 wait states before an MFMA reads an AGPR a VALU wrote
    init = [f'v_accvgpr_write_b32 a{128 + i}, v{i}' for i in range(64)]
    init += [f'v_accvgpr_write_b32 a{i}, 0' for i in range(128)]
    init += ['s_nop 1']
    body = ''.join(f'  "{l}\\n"\n' for l in init)
    text.append("\n// Moves the wave's Q fragments into their AGPRs and zeroes the accumulators.\n")
    text.append('#define TTFA_FWD128_INIT_ASM \\\n' + body.rstrip('\n').replace('\n', ' \\\n') + '\n')
    rd = [f'v_accvgpr_read_b32 v{i}, a{i}' for i in range(128)]
    body = ''.join(f'  "{l}\\n"\n' for l in rd)
    text.append('\n// Reads the O^T accumulators back into v[0:127].\n')
    text.append('#define TTFA_FWD128_READ_ASM \\\n' + body.rstrip('\n').replace('\n', ' \\\n') + '\n')
    return ''.join(text)


def main():
    out = sys.argv[1] if len(sys.argv) > 1 else DEFAULT_OUT
    with open(out, 'w') as f:
        f.write(render(verbose=True))
    print(f'wrote {out}')


if __name__ == '__main__':
    main()
