"""Builds libfletcher_hip.so (gfx950) in-tree from csrc/.

    python longbow-fletcher_amd/build.py [--jobs N]

Each .hip/.cpp file is compiled with hipcc for gfx950 (packed-fp32 ops
disabled, code object v5) and the objects are linked into
longbow-fletcher_amd/lib/libfletcher_hip.so.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
OBJDIR = LIBDIR / "obj"
LIB = LIBDIR / "libfletcher_hip.so"

ARCH = os.environ.get("FLETCHER_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-mcode-object-version=5",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wall", "-Wno-unused-function", f"-I{ROOT / 'include'}"]


# Per-file flags.  gemm.hip: keep MFMA accumulators in architectural VGPRs
# (the accumulator-register form made the allocator copy accumulators every
# K step).
# attention.hip: also no NaN-quieting before every max of the softmax row
# reductions (NaN inputs still propagate through exp2 and the P V products).
PER_FILE = {"gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
            "attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", "-fno-honor-nans"]}


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = OBJDIR / (src.name + ".o")
    cmd = [HIPCC, *COMMON, *PER_FILE.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in (r.stderr or "").splitlines()
                     if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src.name}\n{' '.join(cmd)}\n{errs}")
    if errs.strip():
        sys.stderr.write(errs + "\n")
    return obj


def build(jobs: int | None = None) -> pathlib.Path:
    OBJDIR.mkdir(parents=True, exist_ok=True)
    srcs = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o in objs]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> pathlib.Path:
    """The CPU oracle (test infrastructure) is built by its own Makefile."""
    r = subprocess.run(["make", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed\n{r.stdout}\n{r.stderr}")
    return ROOT / "oracle" / "build" / "libfletcher_oracle.so"


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--no-oracle", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs))
    if not a.no_oracle:
        print(build_oracle())
