"""Compile the HIP sources in csrc/ into lib/libq4nx_hip.so for gfx950.

Each .hip file is compiled to an object in parallel (hipcc, -O3), then linked into one
shared library. `python -m llmnputest_amd.build` rebuilds unconditionally.
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
OBJ = PKG / "_build"
LIB = PKG / "lib" / "libq4nx_hip.so"
ARCH = os.environ.get("Q4NX_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 VALU forms are kept out of generated code on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
# MFMA results in VGPRs: the epilogues read them without v_accvgpr_read copies. The prefill
# contraction keeps its MFMA accumulators in AGPRs instead, which leaves the VGPRs to its
# staged operands and the separately accumulated Q4_1 minimum.
VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
AGPR_ACCUMULATORS: set[str] = set()


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the HIP extension cannot be built")


def _compile(src: Path, verbose: bool) -> Path:
    out = OBJ / (src.stem + ".o")
    extra = [] if src.name in AGPR_ACCUMULATORS else VGPR_FORM
    cmd = [hipcc(), *HIPCC_FLAGS, *extra, "-c", str(src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l and l.strip())
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msgs}")
    if verbose and msgs:
        print(msgs, file=sys.stderr)
    return out


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip and link lib/libq4nx_hip.so. Always rebuilds."""
    OBJ.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
