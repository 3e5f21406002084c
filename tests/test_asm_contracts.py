"""Register and hazard contracts of the hand-written kernels, checked on the compiled
device assembly (CPU only: hipcc cross-compiles gfx950 without a GPU).

Three kernels keep state, or issue products, where the compiler cannot see them:

* the 256-row D = 128 forward (fa_fwd128.hip) and dQ pass (fa_bwd_dq128.hip) hold their
  accumulators and operand fragments in AGPRs between inline-asm statements, outside
  every asm operand list.  That is only correct while the compiler itself never touches
  an AGPR in those kernels: no spill into an AGPR, no copy through one;
* inline-asm MFMAs (mfma32_vacc in fa_bwd.hip, and every product of the generated stage
  streams) are opaque to the compiler's hazard recogniser, so no VALU instruction may
  write one of their source registers within the two wait states before them.

The build compiles these files with the same flags; a toolchain that schedules or
allocates differently fails here instead of corrupting results on the GPU.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

from tinytrain_amd import build as B

CSRC = B.CSRC
WIDE_KERNELS = {"fa_fwd128.hip": "fa_fwd_wide_bf16_kernel",
                "fa_bwd_dq128.hip": "fa_bwd_dq_wide_bf16_kernel"}
_REG = re.compile(r"\b([va])(?:(\d+)|\[(\d+):(\d+)\])")


def _hipcc_or_skip() -> str:
    try:
        return B._hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory) -> dict:
    """{source name: device assembly text} for every csrc/*.hip, built with the
    library's own flags (--cuda-device-only -S)."""
    hipcc = _hipcc_or_skip()
    B._generate()
    out = tmp_path_factory.mktemp("asm")
    procs = {}
    for src in sorted(CSRC.glob("*.hip")):
        dst = out / (src.stem + ".s")
        cmd = [hipcc, *B.HIPCC_FLAGS, f"-I{B.INCLUDE}", f"-I{CSRC}", "--cuda-device-only",
               "-S", str(src), "-o", str(dst)]
        procs[src.name] = (subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT, text=True), dst)
    res = {}
    for name, (p, dst) in procs.items():
        log = p.communicate(timeout=600)[0]
        assert p.returncode == 0, f"hipcc -S failed for {name}:\n{log}"
        res[name] = dst.read_text()
    return res


def _regs(text: str) -> set:
    out = set()
    for m in _REG.finditer(text):
        if m.group(2) is not None:
            out.add((m.group(1), int(m.group(2))))
        else:
            out.update((m.group(1), r) for r in range(int(m.group(3)), int(m.group(4)) + 1))
    return out


def _instructions(asm: str) -> list:
    """(kind, code, inside_inline_asm) per line of code; kind 'L' for labels."""
    res, inasm = [], False
    for line in asm.splitlines():
        if ";;#ASMSTART" in line:
            inasm = True
            continue
        if ";;#ASMEND" in line:
            inasm = False
            continue
        code = line.split(";")[0].strip()
        if not code:
            continue
        if code.endswith(":") or code.startswith(".Lfunc_end"):
            res.append(("L", code, inasm))
        elif not code.startswith("."):
            res.append(("I", code, inasm))
    return res


def _function_body(asm: str, kernel: str) -> str:
    m = re.search(r"^(_Z\S*" + re.escape(kernel) + r"\S*):[^\n]*\n(.*?)^\.Lfunc_end", asm,
                  re.M | re.S)
    assert m, f"{kernel} not found in the assembly"
    return m.group(2)


def _valu_writes_before_inline_mfma(asm: str, wait_states: int = 2) -> list:
    """Inline-asm MFMAs with a VALU write of one of their source registers (A, B or C)
    within ``wait_states`` issue slots before them (s_nop N counts N + 1)."""
    ins = _instructions(asm)
    bad = []
    for i, (kind, code, inasm) in enumerate(ins):
        if kind != "I" or not inasm or not code.startswith("v_mfma"):
            continue
        ops = [o.strip() for o in code.split(None, 1)[1].split(",")]
        src = set().union(*(_regs(o) for o in ops[1:4]))
        ws, j = 0, i - 1
        while ws < wait_states and j >= 0:
            k2, c2, _ = ins[j]
            if k2 == "L":  # a join point: the predecessor is not known here
                break
            op = c2.split()[0]
            if op == "s_nop":
                ws += int(c2.split()[1], 0) + 1
                j -= 1
                continue
            if (op.startswith("v_") and not op.startswith(("v_mfma", "v_cmp", "v_readlane",
                                                            "v_readfirstlane"))):
                parts = c2.split(None, 1)
                dst = _regs(parts[1].split(",")[0]) if len(parts) > 1 else set()
                if dst & src:
                    bad.append((code, c2, ws))
            ws += 1
            j -= 1
    return bad


def test_wide_kernels_touch_no_agpr_outside_their_asm(device_asm):
    for src, kernel in WIDE_KERNELS.items():
        body = _function_body(device_asm[src], kernel)
        outside = [c for k, c, inasm in _instructions(body)
                   if k == "I" and not inasm and re.search(r"\ba\d+\b|\ba\[\d+:\d+\]", c)]
        assert not outside, f"{kernel}: compiler-issued AGPR accesses {outside[:5]}"
        n_asm = sum(1 for k, c, inasm in _instructions(body) if k == "I" and inasm)
        assert n_asm > 1000, f"{kernel}: the generated stream is missing ({n_asm} asm instructions)"


def test_no_spills_and_vgprs_below_accum_offset(device_asm):
    kernels = 0
    for src, asm in device_asm.items():
        for m in re.finditer(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", asm, re.S):
            name, block = m.group(1), m.group(2)
            kernels += 1
            nvgpr = re.search(r"\.amdhsa_next_free_vgpr (\d+)", block)
            acc = re.search(r"\.amdhsa_accum_offset (\d+)", block)
            meta = asm[m.end():]
            info = re.search(r"; NumVgprs: (\d+)\n; NumAgprs: (\d+)\n; TotalNumVgprs: (\d+)\n"
                             r"; ScratchSize: (\d+)", meta)
            assert nvgpr and acc and info, name
            vg, ag, total, scratch = map(int, info.groups())
            assert scratch == 0, f"{src} {name}: scratch {scratch} bytes (spills)"
            assert vg <= int(acc.group(1)), f"{src} {name}: {vg} VGPRs above accum_offset"
            assert total <= 512 and int(nvgpr.group(1)) <= 512, name
    assert kernels >= 25, kernels
    for src, asm in device_asm.items():
        for cnt in re.findall(r"\.(?:v|s)gpr_spill_count:\s+(\d+)", asm):
            assert int(cnt) == 0, f"{src}: register spills"


def test_no_valu_write_before_inline_mfma(device_asm):
    n = 0
    for src, asm in device_asm.items():
        bad = _valu_writes_before_inline_mfma(asm)
        assert not bad, f"{src}: {bad[:3]}"
        n += sum(1 for k, c, inasm in _instructions(asm)
                 if k == "I" and inasm and c.startswith("v_mfma"))
    assert n > 1000  # the generated streams and mfma32_vacc are all inline asm


def test_hazard_check_catches_planted_write():
    # A VALU write of the B operand one slot before the product, and a safe version with
    # two wait states in between.
    hazard = ("\tv_mov_b32 v4, v9\n\t;;#ASMSTART\n"
              "\tv_mfma_f32_32x32x16_bf16 v[16:31], v[0:3], v[4:7], v[16:31]\n\t;;#ASMEND\n")
    safe = ("\tv_mov_b32 v4, v9\n\ts_nop 1\n\t;;#ASMSTART\n"
            "\tv_mfma_f32_32x32x16_bf16 v[16:31], v[0:3], v[4:7], v[16:31]\n\t;;#ASMEND\n")
    acc = ("\tv_accvgpr_write_b32 a2, v9\n\t;;#ASMSTART\n"
           "\tv_mfma_f32_32x32x16_bf16 v[16:31], v[0:3], a[0:3], v[16:31]\n\t;;#ASMEND\n")
    assert len(_valu_writes_before_inline_mfma(hazard)) == 1
    assert _valu_writes_before_inline_mfma(safe) == []
    assert len(_valu_writes_before_inline_mfma(acc)) == 1
