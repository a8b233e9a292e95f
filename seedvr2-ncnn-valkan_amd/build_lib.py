"""Builds libseedvr2_hip.so (gfx950) in-tree with hipcc.

Every HIP/C++ source under csrc/ is compiled to an object in _build/ and the
objects are linked into seedvr2-ncnn-valkan_amd/libseedvr2_hip.so.  Runs on a
machine without a GPU (hipcc cross-compiles for gfx950).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
BUILD = REPO / "_build" / "lib"
LIB = PKG / "libseedvr2_hip.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # packed fp32 ops stay off: some of their forms are unreliable on this part
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]


def sources() -> list[Path]:
    out = []
    for path in sorted(CSRC.rglob("*")):
        if path.suffix in (".hip", ".cpp"):
            out.append(path)
    return out


def _compile(src: Path) -> Path:
    rel = src.relative_to(CSRC)
    obj = BUILD / (str(rel).replace(os.sep, "__") + ".o")
    obj.parent.mkdir(parents=True, exist_ok=True)
    cmd = [HIPCC, *COMMON, "-x", "hip", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(8, len(srcs))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp), *map(str, objs),
           "-L/opt/rocm/lib", "-lhipblaslt", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
