"""Builds tests/cxx/block_runner (the C++ consumer of the layer adapter) with
g++ against include/, libseedvr2_hip.so and the HIP runtime's C API (the
device-chain mode allocates device blobs); no ncnn and no hipcc."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
PKG = REPO / "seedvr2-ncnn-valkan_amd"
OUT = HERE / "_build" / "block_runner"
ROCM = Path("/opt/rocm")


def build(out: Path = OUT) -> Path:
    out.parent.mkdir(parents=True, exist_ok=True)
    if not (PKG / "libseedvr2_hip.so").exists():
        raise RuntimeError("libseedvr2_hip.so is not built")
    # in-tree binaries find the library relative to themselves (the tree moves
    # between machines); others by its absolute path
    try:
        rpath = "$ORIGIN/" + str(Path(*[".."] * len(out.parent.resolve().relative_to(REPO).parts)) / PKG.name)
    except ValueError:
        rpath = str(PKG)
    # the device-chain mode allocates blobs with the HIP runtime's C API
    # (host code: g++ with the AMD platform macro, no hipcc)
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{REPO / 'include'}", f"-I{HERE}", f"-I{ROCM / 'include'}",
           str(HERE / "block_runner.cpp"), "-o", str(out), f"-L{PKG}", "-lseedvr2_hip",
           f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{rpath}", f"-Wl,-rpath,{ROCM / 'lib'}"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return out


if __name__ == "__main__":
    print(build())
