"""Builds tests/cxx/block_runner (the C++ consumer of the layer adapter) with
g++ against include/ and libseedvr2_hip.so; no ncnn and no HIP headers."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
PKG = REPO / "seedvr2-ncnn-valkan_amd"
OUT = HERE / "_build" / "block_runner"


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
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror", f"-I{REPO / 'include'}", f"-I{HERE}",
           str(HERE / "block_runner.cpp"), "-o", str(out), f"-L{PKG}", "-lseedvr2_hip",
           f"-Wl,-rpath,{rpath}"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return out


if __name__ == "__main__":
    print(build())
