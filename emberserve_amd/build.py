"""Builds libember_ops.so (the gfx950 HIP kernels behind the C ABI in include/ember_ops.h).

`python -m emberserve_amd.build` or `build()` compiles every `csrc/*.hip` with hipcc for
gfx950, in parallel, and links the shared library next to this file, where `_lib` loads it.
No GPU is needed: hipcc cross-compiles.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libember_ops.so"
ARCH = "gfx950"

# -ffp-contract=off: a*b+c stays two rounded operations, as in the reference's separate
# element-wise tensor ops (the rope and norm parity depends on it).
# -packed-fp32-ops: keep hipcc from forming packed fp32 instructions.
# -amdgpu-mfma-vgpr-form: MFMA accumulators in ordinary VGPRs, so the decode kernel's
# online-softmax rescale of its accumulators needs no accvgpr copies.
HIP_FLAGS = [
    "-O3", f"--offload-arch={ARCH}", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall", "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")


def build(verbose: bool = False) -> Path:
    """Compiles every kernel source and links `libember_ops.so`; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, workers)) as ex:
        futs = [ex.submit(_compile, s, o) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)  # atomic: a process that already mapped the old file keeps it
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
