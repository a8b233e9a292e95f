"""Builds the C++ consumers under tests/cxx with g++ against include/,
libseedvr2_hip.so and the HIP runtime's C API; no ncnn and no hipcc:
block_runner (the layer adapter, its device-chain mode allocates device
blobs) and dit_step (the 32-block DiT driven through the C ABI alone)."""
from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
PKG = REPO / "seedvr2-ncnn-valkan_amd"
OUT = HERE / "_build" / "block_runner"
DIT_OUT = HERE / "_build" / "dit_step"
ROCM = Path("/opt/rocm")


def _compile(source: Path, out: Path) -> Path:
    out.parent.mkdir(parents=True, exist_ok=True)
    if not (PKG / "libseedvr2_hip.so").exists():
        raise RuntimeError("libseedvr2_hip.so is not built")
    # in-tree binaries find the library relative to themselves (the tree moves
    # between machines); others by its absolute path
    try:
        rpath = "$ORIGIN/" + str(Path(*[".."] * len(out.parent.resolve().relative_to(REPO).parts)) / PKG.name)
    except ValueError:
        rpath = str(PKG)
    # host code calling the HIP runtime's C API: g++ with the AMD platform
    # macro, no hipcc
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-Werror", "-D__HIP_PLATFORM_AMD__",
           f"-I{REPO / 'include'}", f"-I{HERE}", f"-I{ROCM / 'include'}",
           str(source), "-o", str(out), f"-L{PKG}", "-lseedvr2_hip",
           f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{rpath}", f"-Wl,-rpath,{ROCM / 'lib'}"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return out


def build(out: Path = OUT) -> Path:
    return _compile(HERE / "block_runner.cpp", out)


def build_dit_step(out: Path = DIT_OUT) -> Path:
    return _compile(HERE / "dit_step.cpp", out)


if __name__ == "__main__":
    print(build())
    print(build_dit_step())
