"""The generated stage schedules of the backward passes (tinytrain_amd/csrc/
dkdv64_item.inc and dkdv128_item.inc for the dK/dV pass at D = 64 and 128).

The generator inserts the LDS waits and hazard padding that the compiler does not add
inside an asm statement.  This test re-checks the emitted text with an independent
reading of those rules, so a generator change that drops a wait or a nop fails here on
the CPU instead of computing wrong products on the GPU:

  * every register an LDS read fills is used only after an s_waitcnt lgkmcnt(n) whose n
    is at most the number of LDS reads issued after it (reads complete in order);
  * no more than 15 LDS reads are outstanding (the lgkmcnt field);
  * an MFMA result is read or overwritten by VALU / LDS only 12 wait states later, a VALU
    result is read by an MFMA only 2 later, a v_exp result by VALU only 1 later;
  * each variant issues the products, reads and exponentials its blocks need;
  * (D = 128 dK/dV) a symbolic replay of the emitted stream: every register carries a tag
    naming what it holds (a Q/dO row fragment, a transposed fragment, an S or dP partial
    sum after k-step kk, P, dS, packed P/dS), and each product and softmax step checks
    the tags of what it reads, so an LDS read placed after its consumer, or a product
    reading the wrong block's fragments, fails here.
"""

import re
import sys
from pathlib import Path

import pytest

CSRC = Path(__file__).resolve().parent.parent / "tinytrain_amd" / "csrc"


def _gen(name="gen_dkdv64_asm"):
    import importlib
    sys.path.insert(0, str(CSRC))
    try:
        return importlib.import_module(name)
    finally:
        sys.path.pop(0)


def _variants(text, macro="TTFA_DKDV64_STAGE_ASM", label="dkv"):
    """{name: [instruction lines]} from the generated statement."""
    body = re.search(r"#define " + macro + r" \\\n(.*?)\n\n", text, re.S).group(1)
    lines = [m.group(1) for m in re.finditer(r'"(.*?)\\n"', body)]
    out, cur = {}, "FULL"
    out[cur] = []
    for ln in lines:
        m = re.match(r"\.L" + label + r"_(\w+?)_%=:", ln)
        if m:
            cur = m.group(1)
            out[cur] = []
            continue
        if ln.startswith("s_cmp_eq_u32") or ln.startswith("s_cbranch") or ln.startswith("s_branch"):
            continue
        out[cur].append(ln)
    out.pop("end", None)
    return out


def _regs(tok):
    """Register names in one operand token (v7, v[4:7], a[0:3]); operands %N -> itself."""
    m = re.fullmatch(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return [f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)]
    if re.fullmatch(r"[va]\d+", tok):
        return [tok]
    if re.fullmatch(r"%\d+", tok):
        return [tok]
    return []


def _decode(ln):
    """(kind, reads, writes) of one instruction line."""
    op, _, rest = ln.partition(" ")
    toks = [t.strip() for t in rest.split(",")] if rest else []
    toks = [t.split()[0] if t else t for t in toks]
    if op.startswith("ds_read"):
        return "lds", [], _regs(toks[0])
    if op.startswith("v_mfma"):
        dst, a, b, c = toks[:4]
        return "mfma", _regs(a) + _regs(b) + (_regs(c) if c != "0" else []), _regs(dst)
    if op == "v_exp_f32":
        return "trans", _regs(toks[1]), _regs(toks[0])
    if op.startswith("v_cmp"):
        return "valu", [r for t in toks[1:] for r in _regs(t)], ["vcc"]
    if op == "v_mov_b32":
        return "valu", [], _regs(toks[0])
    if op.startswith("v_"):
        reads = [r for t in toks[1:] for r in _regs(t)]
        if op.startswith("v_cndmask"):
            reads.append("vcc")
        return "valu", reads, _regs(toks[0])
    return "other", [], []


def _check_stream(lines):
    ws = 0
    last = {}      # reg -> (ws after writer, kind)
    pending = []   # outstanding LDS reads: sets of registers
    for ln in lines:
        if ln.startswith("s_nop"):
            ws += int(ln.split()[1]) + 1
            continue
        if ln.startswith("s_waitcnt"):
            n = int(re.search(r"lgkmcnt\((\d+)\)", ln).group(1))
            pending = pending[len(pending) - n:] if n < len(pending) else pending
            ws += 1
            continue
        kind, reads, writes = _decode(ln)
        touched = set(reads) | set(writes)
        for w in pending:
            assert not (w & touched), f"{ln!r} touches a register an LDS read is still filling"
        for r in reads + writes:
            if r not in last:
                continue
            at, wk = last[r]
            gap = ws - at
            if wk == "mfma" and kind in ("valu", "trans", "lds"):
                assert gap >= 12, f"{ln!r}: {r} read {gap} wait states after an MFMA wrote it"
            if wk == "mfma" and kind == "mfma" and r not in writes:
                assert gap >= 12, f"{ln!r}: MFMA result {r} used as an operand after {gap}"
            if wk in ("valu", "trans") and kind == "mfma":
                assert gap >= 2, f"{ln!r}: VALU result {r} read by an MFMA after {gap}"
            if wk == "trans" and kind in ("valu", "trans"):
                assert gap >= 1, f"{ln!r}: v_exp result {r} read after {gap}"
        ws += 1
        for r in writes:
            last[r] = (ws, kind)
        if kind == "lds":
            pending.append(set(writes))
            assert len(pending) <= 15, f"{ln!r}: more than 15 LDS reads outstanding"
    assert not pending, "the stream ends with LDS reads outstanding"
    mfma_w = [ws - at for at, k in last.values() if k == "mfma"]
    # the statement ends with the padding a following VALU read of a product needs
    tail = lines[-1]
    pad = int(tail.split()[1]) + 1 if tail.startswith("s_nop") else 0
    assert min(mfma_w) >= 12 or pad > 0


def test_committed_file_is_the_generator_output():
    gen = _gen()
    assert (CSRC / "dkdv64_item.inc").read_text() == gen.render(), \
        "dkdv64_item.inc is stale: run python tinytrain_amd/csrc/gen_dkdv64_asm.py"


@pytest.mark.parametrize("name", ["FULL", "DIAG0", "DIAG1", "DIAG2", "DIAG3"])
def test_stream_rules_and_counts(name):
    gen = _gen()
    var = _variants(gen.render())
    assert set(var) == {"FULL", "DIAG0", "DIAG1", "DIAG2", "DIAG3"}
    lines = var[name]
    _check_stream(lines)
    n_blocks = 4 if name == "FULL" else 4 - int(name[-1])
    count = lambda p: sum(1 for ln in lines if ln.startswith(p))
    assert count("v_mfma") == 16 * n_blocks          # S, dP: 8; dV, dK: 8 per block
    assert count("ds_read") == 32 * n_blocks         # 8 init, 8 rows, 16 transposed halves
    assert count("v_exp_f32") == 32 * n_blocks // 2  # one per score element per lane
    assert count("v_cmp_lt_i32") == (0 if name == "FULL" else 16)  # the diagonal block only
    # every dV/dK product reads a packed P/dS group written by this stream
    assert count("v_cvt_pk_bf16_f32") == 16 * n_blocks


def test_checker_catches_a_dropped_wait_or_nop():
    """The rules above are not vacuous: dropping one LDS wait or one hazard nop from the
    emitted stream makes the check fail."""
    lines = _variants(_gen().render())["FULL"]
    for prefix in ("s_waitcnt lgkmcnt(", "s_nop"):
        i = next(k for k, ln in enumerate(lines) if ln.startswith(prefix) and k > 2)
        with pytest.raises(AssertionError):
            _check_stream(lines[:i] + lines[i + 1:])


# ---- D = 128 dK/dV stage (dkdv128_item.inc) -------------------------------------------
# Register map and operands as the generator's header states them: v[0:15] S of register
# set 0, v[16:31] its dP, v[32:63] set 1; v[64+4kk] Q row fragments, v[96+4kk] dO ones,
# v[128+4db] dO^T, v[144+4db] Q^T; %0..%3 dK^T accumulators, %4..%7 dV^T ones, %8..%15 K
# fragments, %16..%23 V fragments, %24+kk row-read addresses of k-step kk, %32+2db+h
# transposed-read addresses (column block db, 8-row half h), %40 the -LSE/scale rows
# (-Delta at +512).  LDS stage: Q rows at 0, dO rows at +32768, 256 bytes a row, 32-row
# blocks of 8192 bytes.
D128_KK, D128_DB = 8, 4
D128_VARIANTS = {"FULL": [0, 1, 2, 3], "DIAG0": [0, 1, 2, 3], "DIAG1": [1, 2, 3],
                 "DIAG2": [2, 3], "DIAG3": [3]}


def _vrange(tok):
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return list(range(int(m.group(1)), int(m.group(2)) + 1))
    return [int(re.fullmatch(r"v(\d+)", tok).group(1))]


def _set_of(v):
    """(register set, 'S' or 'P', index within the 16) of an S/dP register."""
    rs, r = divmod(v, 32)
    return rs, ("S" if r < 16 else "P"), r % 16


def _dataflow_d128(lines, blocks):
    """Replays one emitted variant on tags; returns a list of errors."""
    reg, acc, errs = {}, {}, []
    for ln in lines:
        if ln.startswith(("s_nop", "s_waitcnt")):
            continue
        m = re.match(r"ds_read_b128 (\S+), %(\d+) offset:(\d+)", ln)
        if m:
            dst, addr, off = _vrange(m.group(1)), int(m.group(2)), int(m.group(3))
            if addr == 40:
                which, r = divmod(off, 512)
                tag = ("init", which, r // 128)
            else:
                tensor, r = divmod(off, 32768)
                if r % 8192:
                    errs.append(f"{ln}: offset inside a block")
                tag = ("row", tensor, r // 8192, addr - 24)
            for i, v in enumerate(dst):
                reg[v] = tag + (i,)
            continue
        m = re.match(r"ds_read_b64_tr_b16 (\S+), %(\d+) offset:(\d+)", ln)
        if m:
            dst, off = _vrange(m.group(1)), int(m.group(3))
            db, h = divmod(int(m.group(2)) - 32, 2)
            tensor, r = divmod(off, 32768)
            row = r // 256
            if row % 16:
                errs.append(f"{ln}: offset inside a 16-row group")
            for i, v in enumerate(dst):
                reg[v] = ("tr", tensor, row // 32, (row % 32) // 16, db, h)
            continue
        m = re.match(r"v_mfma_f32_32x32x16_bf16 (\S+), (\S+), (\S+), (\S+)", ln)
        if m:
            d, a, b, c = m.groups()
            if d.startswith("%"):  # dK^T / dV^T += (Q^T | dO^T) x (packed dS | P)
                n = int(d[1:])
                kind, db = ("dk", n) if n < 4 else ("dv", n - 4)
                A = [reg.get(v) for v in _vrange(a)]
                B = [reg.get(v) for v in _vrange(b)]
                tensor = 0 if kind == "dk" else 1
                if None in A or any(x[0] != "tr" or x[1] != tensor or x[4] != db for x in A) \
                        or [x[5] for x in A] != [0, 0, 1, 1] or len({x[2:4] for x in A}) != 1:
                    errs.append(f"{ln}: A operand {A}")
                    continue
                lb, mg = A[0][2], A[0][3]
                want = "dSk" if kind == "dk" else "Pk"
                if any(x != (want, lb, mg) for x in B):
                    errs.append(f"{ln}: B operand {B}, want {(want, lb, mg)}")
                acc.setdefault((kind, db), []).append((lb, mg))
                continue
            D_, A = _vrange(d), [reg.get(v) for v in _vrange(a)]
            if None in A or any(x[0] != "row" or x[1:4] != A[0][1:4] for x in A):
                errs.append(f"{ln}: A operand {A}")
                continue
            _, tensor, lb, kk = A[0][:4]
            if int(b[1:]) != (8 if tensor == 0 else 16) + kk:
                errs.append(f"{ln}: B operand {b} for k-step {kk}")
            name = "S" if tensor == 0 else "P"
            if {_set_of(v)[1] for v in D_} != {name}:
                errs.append(f"{ln}: destination not a {name} block")
            want = ("init", tensor, lb) if kk == 0 else (name, lb, kk - 1)
            for v in D_:
                x = reg.get(v)
                if x is None or x[:3] != want:
                    errs.append(f"{ln}: C register v{v} holds {x}, want {want}")
                    break
            for v in D_:
                reg[v] = (name, lb, kk)
            continue
        m = re.match(r"v_exp_f32 v(\d+), v(\d+)", ln)
        if m:
            v = int(m.group(1))
            x = reg.get(v)
            if x is None or x[0] != "S" or x[2] != D128_KK - 1:
                errs.append(f"{ln}: exponential of {x}")
            reg[v] = ("p", x[1] if x else None)
            continue
        m = re.match(r"v_mul_f32 v(\d+), v(\d+), v(\d+)", ln)
        if m:  # dS = P * (dP - Delta)
            d, s_, p_ = (int(g) for g in m.groups())
            x, y = reg.get(s_), reg.get(p_)
            if not (x and y and x[0] == "p" and y[0] == "P" and y[2] == D128_KK - 1 and x[1] == y[1]):
                errs.append(f"{ln}: dS from {x} and {y}")
            reg[d] = ("dS", x[1] if x else None)
            continue
        m = re.match(r"v_cvt_pk_bf16_f32 v(\d+), v(\d+), v(\d+)", ln)
        if m:
            d, s0, s1 = (int(g) for g in m.groups())
            rs, name, r = _set_of(d)
            want = "p" if name == "S" else "dS"
            x0, x1 = reg.get(s0), reg.get(s1)
            if not (x0 and x1 and x0[0] == want and x1 == x0):
                errs.append(f"{ln}: packs {x0} and {x1}")
            reg[d] = ("Pk" if name == "S" else "dSk", x0[1] if x0 else None, r // 8)
            continue
    for kind in ("dk", "dv"):
        for db in range(D128_DB):
            want = [(lb, mg) for lb in blocks for mg in range(2)]
            if acc.get((kind, db), []) != want:
                errs.append(f"{kind} column block {db}: contributions {acc.get((kind, db))}, want {want}")
    return errs


def test_d128_committed_file_is_the_generator_output():
    gen = _gen("gen_dkdv128_asm")
    assert (CSRC / "dkdv128_item.inc").read_text() == gen.render(), \
        "dkdv128_item.inc is stale: run python tinytrain_amd/csrc/gen_dkdv128_asm.py"


@pytest.mark.parametrize("name", list(D128_VARIANTS))
def test_d128_stream_rules_counts_and_dataflow(name):
    var = _variants(_gen("gen_dkdv128_asm").render(), "TTFA_DKDV128_STAGE_ASM", "dk128")
    assert set(var) == set(D128_VARIANTS)
    lines = var[name]
    _check_stream(lines)
    n_blocks = len(D128_VARIANTS[name])
    count = lambda p: sum(1 for ln in lines if ln.startswith(p))
    assert count("v_mfma") == 32 * n_blocks           # S, dP: 16; dV, dK: 16 per block
    assert count("ds_read_b128") == 24 * n_blocks     # 8 init, 16 row fragments
    assert count("ds_read_b64_tr_b16") == 32 * n_blocks
    assert count("v_exp_f32") == 16 * n_blocks
    assert count("v_cmp_lt_i32") == (0 if name == "FULL" else 16)
    assert count("v_cvt_pk_bf16_f32") == 16 * n_blocks
    assert _dataflow_d128(lines, D128_VARIANTS[name]) == []


def test_d128_dataflow_check_catches_a_misplaced_read():
    """Moving the first -LSE/scale read of the second block to just after that block's
    first S product (the product then starts from stale registers) fails the replay."""
    lines = _variants(_gen("gen_dkdv128_asm").render(), "TTFA_DKDV128_STAGE_ASM", "dk128")["FULL"]
    inits = [k for k, ln in enumerate(lines) if re.match(r"ds_read_b128 \S+, %40 offset:(128|160|192|224)$", ln)]
    i = inits[0]
    j = next(k for k, ln in enumerate(lines) if k > i and ln.startswith("v_mfma") and ", %8, " in ln)
    moved = lines[:i] + lines[i + 1:j] + [lines[j], lines[i]] + lines[j + 1:]
    assert _dataflow_d128(lines, D128_VARIANTS["FULL"]) == []
    assert _dataflow_d128(moved, D128_VARIANTS["FULL"]) != []


# ---- D = 128 dQ stage (dq128_stage.inc) ------------------------------------------------
# Register map as the generator's header states it: v[0:15] S^T of register set 0,
# v[16:31] its dP^T, v[32:63] set 1; v[64+4kk] K row fragments, v[96+4kk] V ones,
# v[128+16m+4db] K^T fragments; v[160+kk] row-read addresses (%0 ^ 32kk), v[168+i]
# transposed-read addresses (%1 ^ 32i, i = 2db + h).  AGPRs: a[64qg+16db:+15] dQ^T
# accumulators, a[128+32qg+4kk:+3] Q fragments, a[192+32qg+4kk:+3] dO fragments.
# Operands: %2 scale, %3+qg -LSE, %7+qg mask bound, %10+qg the -Delta blocks that start
# the dP^T chains.  LDS stage: K rows at
# 0, V rows at +32768, 256 bytes a row, 32-key blocks of 8192 bytes.


def _agpr_base(tok):
    m = re.fullmatch(r"a\[(\d+):(\d+)\]", tok)
    return int(m.group(1)) if m else None


def _dataflow_dq128(lines):
    """Replays one emitted variant of the dQ stream on tags; returns a list of errors."""
    reg, acc, errs = {}, {}, []
    for ln in lines:
        if ln.startswith(("s_nop", "s_waitcnt")):
            continue
        m = re.match(r"v_(mov|xor)_b32 v(\d+), (?:(\d+), )?(%\d+)$", ln)
        if m and int(m.group(2)) >= 160:
            v, k, base = int(m.group(2)), int(m.group(3) or 0), m.group(4)
            reg[v] = ("addr", base, k)
            continue
        m = re.match(r"ds_read_b128 (\S+), v(\d+) offset:(\d+)", ln)
        if m:
            dst, a, off = _vrange(m.group(1)), int(m.group(2)), int(m.group(3))
            kk = a - 160
            if reg.get(a) != ("addr", "%0", 32 * kk):
                errs.append(f"{ln}: address register holds {reg.get(a)}")
            tensor, r = divmod(off, 32768)
            if r % 8192:
                errs.append(f"{ln}: offset inside a block")
            for i, v in enumerate(dst):
                reg[v] = ("row", tensor, r // 8192, kk)
            continue
        m = re.match(r"ds_read_b64_tr_b16 (\S+), v(\d+) offset:(\d+)", ln)
        if m:
            dst, a, off = _vrange(m.group(1)), int(m.group(2)), int(m.group(3))
            i = a - 168
            if reg.get(a) != ("addr", "%1", 32 * i):
                errs.append(f"{ln}: address register holds {reg.get(a)}")
            db, h = divmod(i, 2)
            row = off // 256
            if off % 256 or (row % 16) // 8 != h:
                errs.append(f"{ln}: offset {off} is not half {h} of a 16-row group")
            for v in dst:
                reg[v] = ("kt", row // 32, (row % 32) // 16, db, h)
            continue
        m = re.match(r"v_mfma_f32_32x32x16_bf16 (\S+), (\S+), (\S+), (\S+)", ln)
        if m:
            d, a, b, c = m.groups()
            if d.startswith("a"):  # dQ^T += K^T dS^T
                qg, db = divmod(_agpr_base(d), 64)
                db //= 16
                A = [reg.get(v) for v in _vrange(a)]
                B = [reg.get(v) for v in _vrange(b)]
                if None in A or any(x[0] != "kt" or x[3] != db for x in A) \
                        or [x[4] for x in A] != [0, 0, 1, 1] or len({x[1:3] for x in A}) != 1:
                    errs.append(f"{ln}: A operand {A}")
                    continue
                lb, mg = A[0][1], A[0][2]
                if any(x != ("dSk", lb, qg, mg) for x in B):
                    errs.append(f"{ln}: B operand {B}, want {('dSk', lb, qg, mg)}")
                acc.setdefault((qg, db), []).append((lb, mg))
                continue
            D_, A = _vrange(d), [reg.get(v) for v in _vrange(a)]
            if None in A or any(x[0] != "row" or x[1:] != A[0][1:] for x in A):
                errs.append(f"{ln}: A operand {A}")
                continue
            _, tensor, lb, kk = A[0]
            bb = _agpr_base(b) - (128 if tensor == 0 else 192)
            qg, bkk = divmod(bb // 4, 8)
            if bkk != kk or not 0 <= qg < 2:
                errs.append(f"{ln}: B operand {b} for k-step {kk}")
            name = "S" if tensor == 0 else "P"
            if {_set_of(v)[1] for v in D_} != {name}:
                errs.append(f"{ln}: destination not a {name} block")
            if kk == 0 and tensor == 0:
                if c != "0":
                    errs.append(f"{ln}: S^T chain does not start at 0")
            elif kk == 0:  # the dP^T chain starts from the row group's -Delta block
                if c != f"%{10 + qg}":
                    errs.append(f"{ln}: dP^T chain of row group {qg} starts from {c}")
            else:
                want = (name, lb, qg, kk - 1)
                bad = [v for v in D_ if reg.get(v) != want]
                if bad:
                    errs.append(f"{ln}: C register v{bad[0]} holds {reg.get(bad[0])}, want {want}")
            for v in D_:
                reg[v] = (name, lb, qg, kk)
            continue
        m = re.match(r"v_fma_f32 v(\d+), v(\d+), %2, %(\d+)$", ln)
        if m:
            v, qg = int(m.group(1)), int(m.group(3)) - 3
            x = reg.get(v)
            if not (x and x[0] == "S" and x[2] == qg and x[3] == 7):
                errs.append(f"{ln}: scaled {x} with row group {qg}'s LSE")
            reg[v] = ("x", x[1] if x else None, qg)
            continue
        m = re.match(r"v_exp_f32 v(\d+), v(\d+)", ln)
        if m:
            v = int(m.group(1))
            x = reg.get(v)
            if not (x and x[0] == "x"):
                errs.append(f"{ln}: exponential of {x}")
            reg[v] = ("p",) + (x[1:] if x else (None, None))
            continue
        m = re.match(r"v_cmp_gt_i32 vcc, (\d+), %(\d+)$", ln)
        if m:
            reg["vcc"] = ("mask", int(m.group(2)) - 7)
            continue
        m = re.match(r"v_cndmask_b32_e64 v(\d+), v(\d+), 0, vcc", ln)
        if m:
            x = reg.get(int(m.group(1)))
            if not (x and x[0] == "p" and reg.get("vcc") == ("mask", x[2])):
                errs.append(f"{ln}: masks {x} with {reg.get('vcc')}")
            continue
        m = re.match(r"v_mul_f32 v(\d+), v(\d+), v(\d+)", ln)
        if m:
            d, s_, p_ = (int(g) for g in m.groups())
            x, y = reg.get(s_), reg.get(p_)
            if not (x and y and x[0] == "p" and y[0] == "P" and y[3] == 7 and x[1:] == y[1:3]):
                errs.append(f"{ln}: dS from {x} and {y}")
            reg[d] = ("dS",) + (x[1:] if x else (None, None))
            continue
        m = re.match(r"v_cvt_pk_bf16_f32 v(\d+), v(\d+), v(\d+)", ln)
        if m:
            d, s0, s1 = (int(g) for g in m.groups())
            x0, x1 = reg.get(s0), reg.get(s1)
            if not (x0 and x0[0] == "dS" and x1 == x0):
                errs.append(f"{ln}: packs {x0} and {x1}")
            reg[d] = ("dSk", x0[1] if x0 else None, x0[2] if x0 else None, (_set_of(d)[2]) // 8)
            continue
        errs.append(f"{ln}: not part of the stream's vocabulary")
    for qg in range(2):
        for db in range(4):
            want = [(lb, mg) for lb in range(4) for mg in range(2)]
            if acc.get((qg, db), []) != want:
                errs.append(f"dQ^T ({qg}, {db}): contributions {acc.get((qg, db))}, want {want}")
    return errs


def _dq128_variants():
    return _variants(_gen("gen_dq128_asm").render(), "TTFA_DQ128_STAGE_ASM", "dq128")


def test_dq128_committed_file_is_the_generator_output():
    gen = _gen("gen_dq128_asm")
    assert (CSRC / "dq128_stage.inc").read_text() == gen.render(), \
        "dq128_stage.inc is stale: run python tinytrain_amd/csrc/gen_dq128_asm.py"


@pytest.mark.parametrize("name", ["FULL", "MASKED"])
def test_dq128_stream_rules_counts_and_dataflow(name):
    var = _dq128_variants()
    assert set(var) == {"FULL", "MASKED"}
    lines = var[name]
    _check_stream(lines)
    count = lambda p: sum(1 for ln in lines if ln.startswith(p))
    assert count("v_mfma") == 8 * 24                  # 8 items: S^T, dP^T 16, dQ^T 8
    assert count("ds_read_b128") == 4 * 16            # K and V rows, once per key block
    assert count("ds_read_b64_tr_b16") == 4 * 16      # K^T halves, once per key block
    assert count("v_exp_f32") == 8 * 16
    assert count("v_cmp_gt_i32") == (0 if name == "FULL" else 8 * 16)
    assert count("v_cvt_pk_bf16_f32") == 8 * 8
    assert _dataflow_dq128(lines) == []


def test_dq128_dataflow_check_catches_a_wrong_row_group():
    """Swapping one product's Q fragment for the other row group's fails the replay, and
    so does dropping one K^T read."""
    lines = _dq128_variants()["FULL"]
    assert _dataflow_dq128(lines) == []
    i = next(k for k, ln in enumerate(lines) if ln.startswith("v_mfma") and ", a[128:131], " in ln)
    swapped = lines[:i] + [lines[i].replace("a[128:131]", "a[160:163]")] + lines[i + 1:]
    assert _dataflow_dq128(swapped) != []
    j = next(k for k, ln in enumerate(lines) if ln.startswith("ds_read_b64_tr_b16"))
    assert _dataflow_dq128(lines[:j] + lines[j + 1:]) != []


# ---- D = 128 forward stage (fwd128_stage.inc) ------------------------------------------


def test_fwd128_committed_file_is_the_generator_output():
    gen = _gen("gen_fwd128_asm")
    assert (CSRC / "fwd128_stage.inc").read_text() == gen.render(), \
        "fwd128_stage.inc is stale: run python tinytrain_amd/csrc/gen_fwd128_asm.py"


@pytest.mark.parametrize("name", ["FULL", "MASKED"])
def test_fwd128_stream_rules_and_counts(name):
    """Waits, hazard padding and instruction counts of the forward stream; the lazy
    rescale blocks are checked as if taken (the conservative reading: the padding after a
    skipped block is then only longer than needed)."""
    var = _variants(_gen("gen_fwd128_asm").render(), "TTFA_FWD128_STAGE_ASM", "fw")
    assert set(var) == {"FULL", "MASKED"}
    lines = var[name]
    _check_stream(lines)
    count = lambda p: sum(1 for ln in lines if ln.startswith(p))
    assert count("v_mfma") == 8 * 16                  # 8 items: S^T 8, PV 8
    assert count("ds_read_b128") == 4 * 8             # K rows, once per key block
    assert count("ds_read_b64_tr_b16") == 4 * 16      # V^T halves, once per key block
    assert count("v_exp_f32") == 8 * (16 + 1)         # P^T, and the rescale factor
    assert count(".Lfr_") == 8                        # one lazy-rescale block per item
    assert count("v_permlane32_swap_b32") == 8        # the row max across the lane halves
    assert count("v_cmp_gt_i32") == (0 if name == "FULL" else 8 * 16)
    assert count("v_cvt_pk_bf16_f32") == 8 * 8
    # every permlane reads its sources 2 wait states after they were written
    for i, ln in enumerate(lines):
        if ln.startswith("v_permlane32_swap_b32"):
            assert lines[i - 1] == "s_nop 1", lines[i - 2:i + 1]


def _dataflow_fwd128(lines):
    """Replays one emitted forward variant on tags (as for the dQ stream): K rows and V^T
    fragments by block, S^T chains by (block, row group, k-step), the row max, P^T and its
    packing, the row-group operands of every softmax step, and each O^T accumulator's
    contributions."""
    reg, acc, errs = {}, {}, []
    cur = None  # (block, row group) whose softmax runs
    for ln in lines:
        if ln.startswith(("s_nop", "s_waitcnt", ".Lfr_")):
            continue
        m = re.match(r"v_(mov|xor)_b32 v(\d+), (?:(\d+), )?(%\d+|0xff800000)$", ln)
        if m and int(m.group(2)) >= 96:
            reg[int(m.group(2))] = ("addr", m.group(4), int(m.group(3) or 0))
            continue
        m = re.match(r"ds_read_b128 (\S+), v(\d+) offset:(\d+)", ln)
        if m:
            a, off = int(m.group(2)), int(m.group(3))
            kk = a - 96
            if reg.get(a) != ("addr", "%4", 32 * kk) or off % 8192 or off >= 32768:
                errs.append(f"{ln}: K row read from {reg.get(a)} at {off}")
            for v in _vrange(m.group(1)):
                reg[v] = ("k", off // 8192, kk)
            continue
        m = re.match(r"ds_read_b64_tr_b16 (\S+), v(\d+) offset:(\d+)", ln)
        if m:
            a, off = int(m.group(2)), int(m.group(3))
            i = a - 104
            db, h = divmod(i, 2)
            row = (off - 32768) // 256
            if reg.get(a) != ("addr", "%5", 32 * i) or off < 32768 or (row % 16) // 8 != h:
                errs.append(f"{ln}: V^T read from {reg.get(a)} at {off}")
            for v in _vrange(m.group(1)):
                reg[v] = ("vt", row // 32, (row % 32) // 16, db, h)
            continue
        m = re.match(r"v_mfma_f32_32x32x16_bf16 (\S+), (\S+), (\S+), (\S+)", ln)
        if m:
            d, a, b, c = m.groups()
            if d.startswith("a"):  # O^T += V^T P^T
                qg, db = divmod(_agpr_base(d), 64)
                db //= 16
                A = [reg.get(v) for v in _vrange(a)]
                B = [reg.get(v) for v in _vrange(b)]
                if None in A or any(x[0] != "vt" or x[3] != db for x in A) \
                        or [x[4] for x in A] != [0, 0, 1, 1] or len({x[1:3] for x in A}) != 1:
                    errs.append(f"{ln}: A operand {A}")
                    continue
                lb, mg = A[0][1], A[0][2]
                if any(x != ("pk", lb, qg, mg) for x in B):
                    errs.append(f"{ln}: B operand {B}, want {('pk', lb, qg, mg)}")
                acc.setdefault((qg, db), []).append((lb, mg))
                continue
            D_, A = _vrange(d), [reg.get(v) for v in _vrange(a)]
            if None in A or any(x[0] != "k" or x != A[0] for x in A):
                errs.append(f"{ln}: A operand {A}")
                continue
            _, lb, kk = A[0]
            qg, bkk = divmod((_agpr_base(b) - 128) // 4, 8)
            if bkk != kk:
                errs.append(f"{ln}: Q fragment k-step {bkk} for K k-step {kk}")
            want = "0" if kk == 0 else None
            if kk == 0 and c != "0":
                errs.append(f"{ln}: chain does not start at 0")
            if kk > 0 and any(reg.get(v) != ("s", lb, qg, kk - 1) for v in D_):
                errs.append(f"{ln}: C holds {reg.get(D_[0])}, want {('s', lb, qg, kk - 1)}")
            for v in D_:
                reg[v] = ("s", lb, qg, kk)
            continue
        m = re.match(r"v_maximum3_f32 v(\d+), v(\d+), v(\d+), v(\d+)", ln)
        if m:
            srcs = [reg.get(int(x)) for x in m.groups()[1:]]
            items = {x[1:3] for x in srcs if x and x[0] in ("s", "mx")}
            if any(x is None or x[0] not in ("s", "mx") or (x[0] == "s" and x[3] != 7) for x in srcs) \
                    or len(items) != 1:
                errs.append(f"{ln}: max over {srcs}")
            else:
                cur = items.pop()
            reg[int(m.group(1))] = ("mx",) + (cur if cur else (None, None))
            continue
        m = re.match(r"v_fma_f32 v(\d+), v(\d+), %6, -%(\d+)$", ln)
        if m:
            v, qg = int(m.group(1)), int(m.group(3))
            x = reg.get(v)
            if not (x and x[0] == "s" and x[3] == 7 and x[2] == qg):
                errs.append(f"{ln}: exponent of {x} with row group {qg}'s max")
            reg[v] = ("x", x[1], x[2]) if x else None
            continue
        m = re.match(r"v_exp_f32 v(\d+), v(\d+)$", ln)
        if m:
            v = int(m.group(1))
            x = reg.get(v)
            if v < 32:
                if not (x and x[0] == "x"):
                    errs.append(f"{ln}: exponential of {x}")
                reg[v] = ("p", x[1], x[2]) if x else None
            continue
        m = re.match(r"v_add_f32 v(\d+), v(\d+), v(\d+)$", ln)
        if m and int(m.group(2)) < 32:
            x = reg.get(int(m.group(2)))
            if not (x and x[0] == "p"):
                errs.append(f"{ln}: row sum of {x}")
            continue
        m = re.match(r"v_add_f32 %(\d+), %(\d+), v(\d+)$", ln)
        if m:
            if not (cur and int(m.group(1)) == 2 + cur[1]):
                errs.append(f"{ln}: row sum into row group {int(m.group(1)) - 2}, item {cur}")
            continue
        m = re.match(r"v_cvt_pk_bf16_f32 v(\d+), v(\d+), v(\d+)", ln)
        if m:
            d, s0, s1 = (int(g) for g in m.groups())
            x0, x1 = reg.get(s0), reg.get(s1)
            if not (x0 and x0[0] == "p" and x1 == x0):
                errs.append(f"{ln}: packs {x0} and {x1}")
            reg[d] = ("pk", x0[1], x0[2], (d % 16) // 8) if x0 else None
            continue
        m = re.match(r"v_add_f32 v\d+, 8\.0, %(\d+)$", ln)
        if m and not (cur and int(m.group(1)) == cur[1]):
            errs.append(f"{ln}: rescale test of row group {m.group(1)}, item {cur}")
    for qg in range(2):
        for db in range(4):
            want = [(lb, mg) for lb in range(4) for mg in range(2)]
            if acc.get((qg, db), []) != want:
                errs.append(f"O^T ({qg}, {db}): contributions {acc.get((qg, db))}, want {want}")
    return errs


@pytest.mark.parametrize("name", ["FULL", "MASKED"])
def test_fwd128_dataflow(name):
    lines = _variants(_gen("gen_fwd128_asm").render(), "TTFA_FWD128_STAGE_ASM", "fw")[name]
    assert _dataflow_fwd128(lines) == []
    # a product with the other row group's Q fragment fails the replay
    i = next(k for k, ln in enumerate(lines) if ln.startswith("v_mfma") and ", a[128:131], " in ln)
    assert _dataflow_fwd128(lines[:i] + [lines[i].replace("a[128:131]", "a[160:163]")] + lines[i + 1:]) != []
