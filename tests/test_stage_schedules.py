"""The generated D = 64 stage schedules of the backward passes (tinytrain_amd/csrc/
dkdv64_item.inc for the dK/dV pass, dq64_stage.inc for the dQ pass).

The generator inserts the LDS waits and hazard padding that the compiler does not add
inside an asm statement.  This test re-checks the emitted text with an independent
reading of those rules, so a generator change that drops a wait or a nop fails here on
the CPU instead of computing wrong products on the GPU:

  * every register an LDS read fills is used only after an s_waitcnt lgkmcnt(n) whose n
    is at most the number of LDS reads issued after it (reads complete in order);
  * no more than 15 LDS reads are outstanding (the lgkmcnt field);
  * an MFMA result is read or overwritten by VALU / LDS only 12 wait states later, a VALU
    result is read by an MFMA only 2 later, a v_exp result by VALU only 1 later;
  * each variant issues the products, reads and exponentials its blocks need.
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


def test_dq_committed_file_is_the_generator_output():
    gen = _gen("gen_dq64_asm")
    assert (CSRC / "dq64_stage.inc").read_text() == gen.render(), \
        "dq64_stage.inc is stale: run python tinytrain_amd/csrc/gen_dq64_asm.py"


@pytest.mark.parametrize("name", ["FULL", "DIAG0", "DIAG1", "DIAG2", "DIAG3", "RAGGED"])
def test_dq_stream_rules_and_counts(name):
    var = _variants(_gen("gen_dq64_asm").render(), "TTFA_DQ64_STAGE_ASM", "dq")
    assert set(var) == {"FULL", "DIAG0", "DIAG1", "DIAG2", "DIAG3", "RAGGED"}
    lines = var[name]
    _check_stream(lines)
    n_blocks = int(name[-1]) + 1 if name.startswith("DIAG") else 4
    count = lambda p: sum(1 for ln in lines if ln.startswith(p))
    assert count("v_mfma") == 12 * n_blocks           # S^T, dP^T: 8; dQ^T: 4 per block
    assert count("ds_read") == 16 * n_blocks          # 8 row fragments, 8 transposed halves
    assert count("v_exp_f32") == 16 * n_blocks
    assert count("v_mov_b32") == 16 * n_blocks        # dP^T starts at -Delta
    masked = {"FULL": 0, "RAGGED": 4}.get(name, 1)
    assert count("v_cmp_gt_i32") == 16 * masked
    assert count("v_cvt_pk_bf16_f32") == 8 * n_blocks
