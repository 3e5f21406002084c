"""Build recipe for libttfa.so (gfx950 only), in-tree.

``python -m tinytrain_amd.build`` compiles every ``csrc/*.hip`` translation unit with
hipcc for ``--offload-arch=gfx950`` in parallel and links ``tinytrain_amd/libttfa.so``.
hipcc cross-compiles, so this runs on a host without a GPU.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIB = PKG / "libttfa.so"
OBJ_DIR = PKG / "_build"

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    # Packed-fp32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: Path, extra: list[str]) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    noise = "is not a recognized feature for this target"
    msgs = [ln for ln in (res.stderr or "").splitlines() if ln.strip() and noise not in ln]
    if msgs:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def _generate() -> None:
    """Rewrites generated sources whose generator output has changed: the D = 64 stage
    schedule of the dK/dV pass (csrc/gen_dkdv64_asm.py -> csrc/dkdv64_item.inc), and the
    D = 128 stage schedule of the dK/dV pass (csrc/gen_dkdv128_asm.py -> csrc/dkdv128_item.inc) and of
    the dQ pass (csrc/gen_dq128_asm.py -> csrc/dq128_stage.inc), and of the D = 128 forward
    (csrc/gen_fwd128_asm.py -> csrc/fwd128_stage.inc)."""
    import importlib
    sys.path.insert(0, str(CSRC))
    try:
        gens = [importlib.import_module(m) for m in ("gen_dkdv64_asm", "gen_dkdv128_asm",
                                                         "gen_dq128_asm", "gen_fwd128_asm")]
    finally:
        sys.path.pop(0)
    for gen in gens:
        text = gen.render()
        out = Path(gen.DEFAULT_OUT)
        if not out.exists() or out.read_text() != text:
            out.write_text(text)


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile all sources and link libttfa.so; returns the library path."""
    _generate()
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    extra = list(extra_flags or [])
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build(verbose=True, extra_flags=sys.argv[1:])
