"""Host-side checks of the block layer's loader (sv2_block_load), no GPU.

Every case here fails while parsing the .param / .bin pair, before any device
call, and must return the reference's codes: -1 for a graph or parameter
problem (SeedVR2DiTBlock::load_param, seedvr2_dit_block.cpp:643-655), -100
for a weight stream that ends early (load_model, :657-688).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import ncnn_files as nf


def _load(hip, param, binf):
    h = ctypes.c_void_p()
    rc = hip.load().sv2_block_load(str(param).encode(), str(binf).encode(), hip.F32, ctypes.byref(h))
    msg = hip.load().sv2_last_error().decode()
    assert not h.value, "no block may be created when loading fails"
    return rc, msg


def _small_files(tmp_path, storage="fp16", truncate=0, **param_kw):
    dim, hidden = 128, 64
    rng = np.random.default_rng(0)
    w = nf.random_weights(rng, dim, hidden, shared=False)
    param = tmp_path / "blk.ncnn.param"
    binf = tmp_path / "blk.ncnn.bin"
    kw = dict(dim=dim, heads=1, mlp_hidden=hidden)
    kw.update(param_kw)
    nf.write_param(param, **kw)
    nf.write_bin(binf, w, shared=False, storage=storage)
    if truncate:
        data = binf.read_bytes()
        binf.write_bytes(data[:-truncate])
    return param, binf


def test_missing_files(hip, tmp_path):
    rc, msg = _load(hip, tmp_path / "none.param", tmp_path / "none.bin")
    assert rc == hip.SV2_EINVAL and "cannot open" in msg


def test_bad_magic(hip, tmp_path):
    param, binf = _small_files(tmp_path)
    param.write_text(param.read_text().replace("7767517", "7767518", 1))
    rc, msg = _load(hip, param, binf)
    assert rc == hip.SV2_EINVAL and "magic" in msg


def test_no_block_layer(hip, tmp_path):
    param, binf = _small_files(tmp_path)
    param.write_text(param.read_text().replace("SeedVR2DiTBlock", "SeedVR2DiTInput"))
    rc, msg = _load(hip, param, binf)
    assert rc == hip.SV2_EINVAL and "no SeedVR2DiTBlock" in msg


def test_blob_count(hip, tmp_path):
    param = tmp_path / "b.param"
    param.write_text("7767517\n1 3\nSeedVR2DiTBlock b 2 1 vid txt out 4=128 5=1 7=64\n")
    binf = tmp_path / "b.bin"
    binf.write_bytes(b"")
    rc, msg = _load(hip, param, binf)
    assert rc == hip.SV2_EINVAL and "4 bottoms" in msg


def test_truncated_layer_line(hip, tmp_path):
    param = tmp_path / "b.param"
    param.write_text("7767517\n2 4\nSeedVR2DiTBlock b 4 2 vid txt emb\n")
    rc, msg = _load(hip, param, tmp_path / "b.bin")
    assert rc == hip.SV2_EINVAL


def test_dim_not_heads_times_head_dim(hip, tmp_path):
    # load_param's only check (seedvr2_dit_block.cpp:652-653)
    param, binf = _small_files(tmp_path, heads=2)
    rc, msg = _load(hip, param, binf)
    assert rc == hip.SV2_EINVAL and "heads * head_dim" in msg


def test_head_dim_unsupported(hip, tmp_path):
    param, binf = _small_files(tmp_path, dim=128, heads=2, head_dim=64)
    rc, _ = _load(hip, param, binf)
    assert rc == hip.SV2_EUNSUPPORTED


@pytest.mark.parametrize("storage", ["fp16", "fp32", "fp32c", "quant"])
def test_truncated_weights(hip, tmp_path, storage):
    # one byte short: the rope freqs record (the last one) cannot be read
    param, binf = _small_files(tmp_path, storage=storage, truncate=1)
    rc, msg = _load(hip, param, binf)
    assert rc == hip.SV2_EDEVICE and "ended early" in msg


def test_int8_records_rejected(hip, tmp_path):
    param, binf = _small_files(tmp_path)
    data = bytearray(binf.read_bytes())
    # first tagged record follows the six ada vectors of width 128
    off = 6 * 128 * 4
    assert int.from_bytes(data[off:off + 4], "little") == nf.TAG_FP16
    data[off:off + 4] = (0x000D4B38).to_bytes(4, "little")
    binf.write_bytes(bytes(data))
    rc, msg = _load(hip, param, binf)
    assert rc == hip.SV2_EDEVICE and "int8" in msg


def test_param_values(tmp_path):
    """The writer's .param reads back with the values the block expects
    (float params such as 8=1e-05 and the optional ids 9-13)."""
    param = tmp_path / "p.param"
    nf.write_param(param, index=7, shared=True, last=True, shifted=True, extra="9=2 10=8 11=10 12=1 13=0")
    lines = param.read_text().splitlines()
    assert lines[0] == "7767517"
    assert lines[1] == "5 6"
    block = lines[-1].split()
    assert block[:4] == ["SeedVR2DiTBlock", "p", "4", "2"]
    kv = dict(item.split("=") for item in block[10:])
    assert kv == {"0": "7", "1": "1", "2": "1", "3": "1", "4": "2560", "5": "20", "6": "128", "7": "6912",
                  "8": "1e-05", "9": "2", "10": "8", "11": "10", "12": "1", "13": "0"}


def test_bin_record_sizes(tmp_path):
    """Byte layout of the .bin against the exporter's record sizes
    (raw fp32 vectors; tag + fp16 values padded to 4 bytes)."""
    dim, hidden = 128, 66  # 66 * 128 fp16 values: no padding; out proj too
    rng = np.random.default_rng(1)
    w = nf.random_weights(rng, dim, hidden, shared=True)
    binf = tmp_path / "w.bin"
    nf.write_bin(binf, w, shared=True, storage="fp16")
    mats = [3 * dim * dim, dim * dim, hidden * dim, hidden * dim, dim * hidden]
    expect = 6 * dim * 4 + sum(4 + ((2 * n + 3) // 4) * 4 for n in mats) + (dim + 2 * 128) * 4 + 21 * 4
    assert binf.stat().st_size == expect
    # odd fp16 counts are padded
    tiny = tmp_path / "t.bin"
    with open(tiny, "wb") as f:
        dec = nf._tagged(f, np.array([1.0, -2.0, 3.0], np.float32), "fp16")
    assert tiny.stat().st_size == 4 + 8
    assert dec.tolist() == [1.0, -2.0, 3.0]


def test_quantise_roundtrip():
    v = np.linspace(-1, 1, 1000, dtype=np.float32)
    table, idx = nf.quantise(v)
    assert table.shape == (256,) and idx.dtype == np.uint8
    assert np.abs(table[idx] - v).max() <= (2.0 / 255) / 2 + 1e-6


def test_runner_fills():
    """The reference runner's deterministic fills (dit_block_vulkan_runner.cpp:43-53, :80-113)."""
    f = nf.runner_fill(4, 3, 100)
    # idx 0..11 + 100: (100 % 11) = 1 -> (1 - 5) * 0.1
    assert f[0, 0] == np.float32(-0.4)
    assert f.reshape(-1)[10] == np.float32((110 % 11 - 5) * np.float32(0.1))
    w = nf.runner_weights(128, 128, 128, shared=True)
    assert set(w) == {"vid", "freqs"}
    assert w["vid"]["w_qkv"].shape == (384, 128)
    assert w["vid"]["w_proj"][0, 0] == np.float32(0.005) * np.float32(7 % 7 - 3)
    assert w["vid"]["b_proj"][1] == np.float32(0.01) * np.float32((1 + 7) % 5 - 2)


# --- the DiT heads and the model directory loader -------------------------

def _head_load(hip, fn, param, binf):
    h = ctypes.c_void_p()
    rc = getattr(hip.load(), fn)(str(param).encode(), str(binf).encode(), hip.F32, ctypes.byref(h))
    assert not h.value
    return rc, hip.load().sv2_last_error().decode()


def _head_files(tmp_path, which, **kw):
    rng = np.random.default_rng(2)
    param, binf = tmp_path / f"{which}.param", tmp_path / f"{which}.bin"
    if which == "input":
        w = nf.random_input_weights(rng, 16, video_channels=2, text_channels=8, sinusoidal_dim=8)
        nf.write_input_files(param, binf, w, dim=16, video_channels=2, text_channels=8, sinusoidal_dim=8, **kw)
    else:
        w = nf.random_output_weights(rng, 16, output_channels=2)
        nf.write_output_files(param, binf, w, dim=16, output_channels=2, **kw)
    return param, binf


def test_input_head_param_checks(hip, tmp_path):
    param, binf = _head_files(tmp_path, "input")
    # load_param rejects embedding_dim != 6 * dim (seedvr2_dit_input.cpp:214)
    param.write_text(param.read_text().replace("4=96", "4=95"))
    rc, msg = _head_load(hip, "sv2_dit_input_load", param, binf)
    assert rc == hip.SV2_EINVAL and "embedding_dim" in msg
    param.write_text(param.read_text().replace("4=95", "4=96").replace("3=8", "3=7"))
    rc, _ = _head_load(hip, "sv2_dit_input_load", param, binf)
    assert rc == hip.SV2_EINVAL


def test_input_head_truncated(hip, tmp_path):
    param, binf = _head_files(tmp_path, "input")
    binf.write_bytes(binf.read_bytes()[:-4])
    rc, msg = _head_load(hip, "sv2_dit_input_load", param, binf)
    assert rc == hip.SV2_EDEVICE and "ended early" in msg


def test_output_head_checks(hip, tmp_path):
    param, binf = _head_files(tmp_path, "output")
    binf.write_bytes(binf.read_bytes()[:-1])
    rc, msg = _head_load(hip, "sv2_dit_output_load", param, binf)
    assert rc == hip.SV2_EDEVICE and "ended early" in msg
    param.write_text(param.read_text().replace("SeedVR2DiTOutput", "SeedVR2DiTInput"))
    rc, msg = _head_load(hip, "sv2_dit_output_load", param, binf)
    assert rc == hip.SV2_EINVAL


def test_model_dir_missing_file(hip, tmp_path):
    """SeedVR2DiT::load checks all 34 file pairs before loading any
    (src/model/dit.cpp:122-134)."""
    _head_files(tmp_path, "input")
    h = ctypes.c_void_p()
    rc = hip.load().sv2_dit_load(str(tmp_path).encode(), hip.F32, ctypes.byref(h))
    assert rc == hip.SV2_EINVAL and not h.value
    assert "seedvr2_dit_input.ncnn.param" in hip.load().sv2_last_error().decode()
