"""The DiT driven from C++ through the C ABI alone (tests/cxx/dit_step, built
by build()): a process without torch creates the input head, the 32 blocks
and the output head from device weights and runs sv2_dit_forward, as a C++
integration holds the model resident (src/model/dit.cpp:120-174, :281-383).
The forward must finish with a finite output, and the process must map the
libhipblaslt the library links (ROCm's), not a copy bundled with torch."""
from __future__ import annotations

import json
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "cxx" / "_build" / "dit_step"


@pytest.mark.parametrize("fused", [0, 1])
def test_dit_from_cxx(fused):
    assert EXE.exists(), "tests/cxx/_build/dit_step is not built (build() compiles it)"
    # a small latent grid (the weights are the full model's): 2 x 16 x 16 ->
    # patched 2 x 8 x 8, 8 text tokens
    cmd = [str(EXE), "--frames", "2", "--height", "16", "--width", "16", "--text", "8", "--steps", "1",
           "--warmup", "0", "--fused", str(fused)]
    print("[dit_step]", " ".join(cmd[1:]), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr
    rep = json.loads([ln for ln in proc.stdout.splitlines() if ln.startswith("{")][-1])
    print(rep, flush=True)
    assert rep["finite"]
    assert rep["hipblaslt"], "no libhipblaslt mapped"
    assert "torch" not in rep["hipblaslt"], rep["hipblaslt"]
