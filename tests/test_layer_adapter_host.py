"""The C++ layer boundary, on the host: tests/cxx/block_runner (a consumer
that includes include/seedvr2_dit_block_layer.h and links libseedvr2_hip.so,
with no ncnn and no HIP headers) is compiled here, and its --load-only mode
drives SeedVR2DiTBlock::load_param / load_model (seedvr2_dit_block.cpp:
643-688) through the adapter on exported blocks: every parameter id, every
ModelBin record type, shared and per-branch weights, and the error codes of
a bad parameter set or a short weight stream."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import ncnn_files as nf

sys.path.insert(0, str(Path(__file__).resolve().parent / "cxx"))
import build_runner  # noqa: E402


@pytest.fixture(scope="module")
def runner(tmp_path_factory):
    if not (build_runner.PKG / "libseedvr2_hip.so").exists():
        pytest.skip("libseedvr2_hip.so not built")
    return build_runner.build(tmp_path_factory.mktemp("cxx") / "block_runner")


def run(runner, *args):
    return subprocess.run([str(runner), *map(str, args)], capture_output=True, text=True, timeout=120)


def params_of(stdout: str) -> dict:
    line = next(l for l in stdout.splitlines() if l.startswith("params "))
    return {int(k): v for k, v in (kv.split("=") for kv in line.split()[1:])}


def test_usage(runner):
    r = run(runner)
    assert r.returncode == 2 and "usage" in r.stderr


@pytest.mark.parametrize("storage", ["fp16", "fp32", "fp32c", "quant"])
@pytest.mark.parametrize("shared", [False, True], ids=["branches", "shared"])
def test_load_only(runner, tmp_path, storage, shared):
    rng = np.random.default_rng(3)
    w = nf.random_weights(rng, 256, 512, shared=shared)
    param, binf = tmp_path / "b.param", tmp_path / "b.bin"
    nf.write_param(param, index=11, shared=shared, last=shared, shifted=True, dim=256, heads=2, mlp_hidden=512,
                   eps="2.5e-06", extra="9=2 10=8 11=10 12=1 13=0 14=1")
    nf.write_bin(binf, w, shared=shared, storage=storage)
    r = run(runner, "--load-only", param, binf)
    assert r.returncode == 0, r.stderr
    p = params_of(r.stdout)
    assert [int(p[i]) for i in (0, 1, 2, 3, 4, 5, 6, 7)] == [11, int(shared), int(shared), 1, 256, 2, 128, 512]
    assert float(p[8]) == np.float32(2.5e-6)
    assert [int(p[i]) for i in range(9, 15)] == [2, 8, 10, 1, 0, 1]
    assert "trailing_bytes=0" in r.stdout


def test_load_only_defaults(runner, tmp_path):
    """Ids 9-14 absent: the reference semantics (adaptive windows, reference
    RoPE, q/k norm on, library GEMMs)."""
    param, binf = tmp_path / "b.param", tmp_path / "b.bin"
    nf.write_param(param, dim=256, heads=2, mlp_hidden=512)
    nf.write_bin(binf, nf.random_weights(np.random.default_rng(4), 256, 512, shared=False), shared=False)
    r = run(runner, "--load-only", param, binf)
    assert r.returncode == 0, r.stderr
    p = params_of(r.stdout)
    assert [int(p[i]) for i in range(9, 15)] == [0, 0, 0, 0, 1, 0]
    assert float(p[8]) == np.float32(1e-5)


def test_load_param_rejects_bad_dim(runner, tmp_path):
    """load_param returns -1 when dim != heads * head_dim (:654)."""
    param, binf = tmp_path / "b.param", tmp_path / "b.bin"
    nf.write_param(param, dim=256, heads=3, mlp_hidden=512)
    binf.write_bytes(b"")
    r = run(runner, "--load-only", param, binf)
    assert r.returncode == 4 and "failed to load block param" in r.stderr


@pytest.mark.parametrize("cut", [4, 1000, 30000])
def test_load_model_rejects_short_stream(runner, tmp_path, cut):
    """load_model returns -100 for a record that ends early (:682-687)."""
    param, binf = tmp_path / "b.param", tmp_path / "b.bin"
    nf.write_param(param, dim=256, heads=2, mlp_hidden=512)
    nf.write_bin(binf, nf.random_weights(np.random.default_rng(5), 256, 512, shared=False), shared=False)
    data = binf.read_bytes()
    binf.write_bytes(data[:-cut])
    r = run(runner, "--load-only", param, binf)
    assert r.returncode == 4 and "failed to load block model" in r.stderr


def test_unregistered_layer_type(runner, tmp_path):
    param, binf = tmp_path / "b.param", tmp_path / "b.bin"
    param.write_text("7767517\n1 1\nSomethingElse x 0 1 y\n")
    binf.write_bytes(b"")
    r = run(runner, "--load-only", param, binf)
    assert r.returncode == 4 and "not exists or registered" in r.stderr


def test_missing_input_file(runner, tmp_path):
    """Full command line with an input that cannot be read: exit 3 once the
    model has loaded, or 4 when no device can take the weights."""
    param, binf = tmp_path / "b.param", tmp_path / "b.bin"
    nf.write_param(param, dim=256, heads=2, mlp_hidden=512)
    nf.write_bin(binf, nf.random_weights(np.random.default_rng(6), 256, 512, shared=False), shared=False)
    r = run(runner, param, binf, tmp_path / "none.f32", 8, tmp_path / "none.f32", 2, tmp_path / "none.f32",
            1, 2, 4, tmp_path / "vo.f32", tmp_path / "to.f32")
    assert r.returncode in (3, 4), (r.returncode, r.stderr)
