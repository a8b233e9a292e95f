"""Writers of one SeedVR2DiTBlock as an ncnn .param / .bin pair, for tests.

The layout follows the reference's exporter (tools/export_seedvr2_dit_ncnn.py:
166-187 for the .param graph, :120-150 and :222-236 for the .bin records):
Input layers for vid/txt/emb/vid_shape, then the block line with params
0-8; per branch ("vid" and "txt", or one shared branch) six raw fp32 ada
vectors, the tagged QKV and proj matrices, the raw proj bias and q/k norm
weights, the tagged gate/in/out MLP matrices; the 21 raw rope freqs last.

`storage` picks the type-0 record of the matrices:
  "fp16"   tag 0x01306B47 + fp16 values padded to 4 bytes (the exporter's default)
  "fp32"   tag 0 + fp32 values (the exporter's --storage fp32)
  "fp32c"  tag 0x0002C056 + fp32 values
  "quant"  a non-zero untagged flag + 256-entry fp32 table + uint8 indices
Also reproduces the deterministic synthetic blocks of the reference's block
runner (tests/dit_block_vulkan_runner.cpp:43-113, :213-218), written with
explicit type-0 tags.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

from parity import reference_freqs

TAG_FP16 = 0x01306B47
TAG_FP32C = 0x0002C056

BRANCH_FIELDS = ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate",
                 "w_qkv", "w_proj", "b_proj", "norm_q", "norm_k", "w_gate", "w_in", "w_out")
MATRICES = ("w_qkv", "w_proj", "w_gate", "w_in", "w_out")


def write_param(path: Path, *, index=0, shared=False, last=False, shifted=False, dim=2560, heads=20,
                head_dim=128, mlp_hidden=6912, eps="1e-05", extra: str = "") -> None:
    inputs = ("vid", "txt", "emb", "vid_shape")
    outputs = ("vid_out", "txt_out")
    params = (f"0={index} 1={int(shared)} 2={int(last)} 3={int(shifted)} 4={dim} 5={heads} "
              f"6={head_dim} 7={mlp_hidden} 8={eps}" + (f" {extra}" if extra else ""))
    lines = [f"Input input_{n} 0 1 {n}" for n in inputs]
    lines.append(" ".join(["SeedVR2DiTBlock", path.stem, "4", "2", *inputs, *outputs, params]))
    path.write_text(f"7767517\n{len(lines)} {len(inputs) + len(outputs)}\n" + "\n".join(lines) + "\n")


def quantise(values: np.ndarray):
    """256-level table quantisation: returns (table [256] f32, indices u8)."""
    v = values.astype(np.float32).reshape(-1)
    lo, hi = float(v.min()), float(v.max())
    table = np.linspace(lo, hi, 256, dtype=np.float32) if hi > lo else np.full(256, lo, np.float32)
    step = (hi - lo) / 255 if hi > lo else 1.0
    idx = np.clip(np.rint((v - lo) / step), 0, 255).astype(np.uint8)
    return table, idx


def _tagged(out, values: np.ndarray, storage: str) -> np.ndarray:
    """Writes one type-0 record; returns the values a reader decodes from it."""
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    if storage == "fp16":
        h = v.astype(np.float16)
        out.write(struct.pack("<I", TAG_FP16))
        raw = h.tobytes()
        out.write(raw + b"\0" * ((-len(raw)) % 4))
        return h.astype(np.float32)
    if storage in ("fp32", "fp32c"):
        out.write(struct.pack("<I", 0 if storage == "fp32" else TAG_FP32C))
        out.write(v.astype("<f4").tobytes())
        return v
    if storage == "quant":
        table, idx = quantise(v)
        out.write(struct.pack("<I", 1))  # any non-zero flag that is not a known tag
        out.write(table.astype("<f4").tobytes())
        raw = idx.tobytes()
        out.write(raw + b"\0" * ((-len(raw)) % 4))
        return table[idx]
    raise ValueError(storage)


def write_bin(path: Path, weights: dict, *, shared: bool, storage: str = "fp16") -> dict:
    """weights: {"vid": {field: array}, "txt": {...}, "freqs": [21]}.  Returns
    the weights as a reader decodes them (same structure, fp32)."""
    decoded = {}
    with open(path, "wb") as out:
        for name in (("vid",) if shared else ("vid", "txt")):
            src = weights[name]
            dec = {}
            for f in BRANCH_FIELDS:
                if f in MATRICES:
                    dec[f] = _tagged(out, src[f], storage).reshape(np.shape(src[f]))
                else:
                    v = np.ascontiguousarray(src[f], dtype=np.float32)
                    out.write(v.astype("<f4").tobytes())
                    dec[f] = v
            decoded[name] = dec
        fr = np.ascontiguousarray(weights["freqs"], dtype=np.float32).reshape(-1)
        out.write(fr.astype("<f4").tobytes())
        decoded["freqs"] = fr
    return decoded


def shapes(dim: int, mlp_hidden: int, head_dim: int = 128) -> dict:
    return {
        "attn_shift": (dim,), "attn_scale": (dim,), "attn_gate": (dim,),
        "mlp_shift": (dim,), "mlp_scale": (dim,), "mlp_gate": (dim,),
        "w_qkv": (3 * dim, dim), "w_proj": (dim, dim), "b_proj": (dim,),
        "norm_q": (head_dim,), "norm_k": (head_dim,),
        "w_gate": (mlp_hidden, dim), "w_in": (mlp_hidden, dim), "w_out": (dim, mlp_hidden),
    }


def random_weights(rng: np.random.Generator, dim: int, mlp_hidden: int, *, shared: bool, std=0.02,
                   fp16_values=True) -> dict:
    """N(0, std^2) weights, q/k norm weights U(0.5, 1.5), reference rope freqs.
    fp16_values rounds every value to fp16 so fp16 and fp32 compute modes see
    identical weights."""
    sh = shapes(dim, mlp_hidden)

    def branch():
        d = {}
        for f, s in sh.items():
            if f in ("norm_q", "norm_k"):
                v = rng.uniform(0.5, 1.5, size=s)
            else:
                v = rng.standard_normal(size=s, dtype=np.float32) * np.float32(std)
            v = v.astype(np.float32)
            d[f] = v.astype(np.float16).astype(np.float32) if fp16_values else v
        return d

    w = {"vid": branch()}
    if not shared:
        w["txt"] = branch()
    w["freqs"] = reference_freqs()
    return w


# --- the reference block runner's synthetic cases -------------------------

# (dim, heads, head_dim, mlp_hidden, T, H, W, text_len, shared, last, shifted, name)
RUNNER_CASES = [
    (128, 1, 128, 128, 2, 2, 2, 3, False, False, False, "basic"),
    (128, 1, 128, 128, 2, 2, 2, 3, False, False, True, "shifted"),
    (128, 1, 128, 128, 1, 1, 1, 2, True, True, False, "last_layer_shared_single_patch"),
    (256, 2, 128, 128, 3, 2, 2, 4, False, False, False, "dim256_heads2_T3"),
]


def runner_fill(cols: int, rows: int, seed_offset: int) -> np.ndarray:
    """fill() of the runner: ((idx + seed) % 11 - 5) * 0.1 in row-major order."""
    idx = np.arange(rows * cols, dtype=np.int64) + seed_offset
    return ((idx % 11 - 5).astype(np.float32) * np.float32(0.1)).reshape(rows, cols)


def _runner_vec(n: int, seed: int) -> np.ndarray:
    i = np.arange(n, dtype=np.int64) + seed
    return np.float32(0.01) * (i % 9 - 4).astype(np.float32)


def _runner_ip(in_: int, out: int, seed: int):
    i = np.arange(in_ * out, dtype=np.int64) + seed
    w = (np.float32(0.005) * (i % 7 - 3).astype(np.float32)).reshape(out, in_)
    j = np.arange(out, dtype=np.int64) + seed
    b = np.float32(0.01) * (j % 5 - 2).astype(np.float32)
    return w, b


def runner_weights(dim: int, head_dim: int, mlp_hidden: int, shared: bool) -> dict:
    def branch(base):
        d = {}
        for k, f in enumerate(BRANCH_FIELDS[:6]):
            d[f] = _runner_vec(dim, base + k)
        d["w_qkv"], _ = _runner_ip(dim, 3 * dim, base + 6)
        d["w_proj"], d["b_proj"] = _runner_ip(dim, dim, base + 7)
        d["norm_q"] = _runner_vec(head_dim, base + 8)
        d["norm_k"] = _runner_vec(head_dim, base + 9)
        d["w_gate"], _ = _runner_ip(dim, mlp_hidden, base + 10)
        d["w_in"], _ = _runner_ip(dim, mlp_hidden, base + 11)
        d["w_out"], _ = _runner_ip(mlp_hidden, dim, base + 12)
        return d

    w = {"vid": branch(0)}
    if not shared:
        w["txt"] = branch(50)
    w["freqs"] = _runner_vec(21, 100)
    return w


def runner_inputs(dim: int, T: int, H: int, W: int, text_len: int):
    vid = runner_fill(dim, T * H * W, 0)
    txt = runner_fill(dim, text_len, 100)
    emb = runner_fill(dim * 6, 1, 200).reshape(-1)
    return vid, txt, emb


# --- the DiT input / output heads and a whole model directory -------------

INPUT_FIELDS = ("w_vid", "b_vid", "w_txt", "b_txt", "w_time_in", "b_time_in", "w_time_hid", "b_time_hid",
                "w_time_out", "b_time_out")
OUTPUT_FIELDS = ("norm_weight", "shift", "scale", "w_proj", "b_proj")


def _write_layer_param(path: Path, layer_type: str, inputs, outputs, params: str) -> None:
    lines = [f"Input input_{n} 0 1 {n}" for n in inputs]
    lines.append(" ".join([layer_type, path.stem, str(len(inputs)), str(len(outputs)), *inputs, *outputs, params]))
    path.write_text(f"7767517\n{len(lines)} {len(set(inputs) | set(outputs))}\n" + "\n".join(lines) + "\n")


def write_input_files(param: Path, binf: Path, weights: dict, *, dim, video_channels=33, text_channels=5120,
                      sinusoidal_dim=256, storage="fp16") -> dict:
    """tools/export_seedvr2_dit_ncnn.py:251-279: each InnerProduct writes its
    tagged matrix, then its raw bias.  Returns the decoded weights."""
    _write_layer_param(param, "SeedVR2DiTInput", ("vid", "txt", "timestep", "vid_shape"),
                       ("vid_out", "txt_out", "emb", "patched_shape"),
                       f"0={dim} 1={video_channels} 2={text_channels} 3={sinusoidal_dim} 4={6 * dim}")
    dec = {}
    with open(binf, "wb") as out:
        for f in INPUT_FIELDS:
            a = np.ascontiguousarray(weights[f], dtype=np.float32)
            if f.startswith("w_"):
                dec[f] = _tagged(out, a, storage).reshape(a.shape)
            else:
                out.write(a.astype("<f4").tobytes())
                dec[f] = a
    return dec


def write_output_files(param: Path, binf: Path, weights: dict, *, dim, output_channels=16, eps="1e-05",
                       storage="fp16") -> dict:
    """tools/export_seedvr2_dit_ncnn.py:282-297: norm weight, out shift, out
    scale (raw), the tagged projection matrix, its raw bias."""
    _write_layer_param(param, "SeedVR2DiTOutput", ("vid", "emb", "vid_shape"), ("vid_out", "output_shape"),
                       f"0={dim} 1={output_channels} 2={eps}")
    dec = {}
    with open(binf, "wb") as out:
        for f in OUTPUT_FIELDS:
            a = np.ascontiguousarray(weights[f], dtype=np.float32)
            if f == "w_proj":
                dec[f] = _tagged(out, a, storage).reshape(a.shape)
            else:
                out.write(a.astype("<f4").tobytes())
                dec[f] = a
    return dec


def random_input_weights(rng, dim, *, video_channels=33, text_channels=5120, sinusoidal_dim=256, std=0.02):
    shp = {"w_vid": (dim, 4 * video_channels), "b_vid": (dim,), "w_txt": (dim, text_channels), "b_txt": (dim,),
           "w_time_in": (dim, sinusoidal_dim), "b_time_in": (dim,), "w_time_hid": (dim, dim),
           "b_time_hid": (dim,), "w_time_out": (6 * dim, dim), "b_time_out": (6 * dim,)}
    return {k: (rng.standard_normal(s, dtype=np.float32) * np.float32(std)).astype(np.float16).astype(np.float32)
            for k, s in shp.items()}


def random_output_weights(rng, dim, *, output_channels=16, std=0.02):
    w = {"norm_weight": rng.uniform(0.5, 1.5, dim).astype(np.float32),
         "shift": rng.standard_normal(dim, dtype=np.float32) * np.float32(std),
         "scale": rng.standard_normal(dim, dtype=np.float32) * np.float32(std),
         "w_proj": rng.standard_normal((4 * output_channels, dim), dtype=np.float32) * np.float32(std),
         "b_proj": rng.standard_normal(4 * output_channels, dtype=np.float32) * np.float32(std)}
    return {k: v.astype(np.float16).astype(np.float32) for k, v in w.items()}


def block_flags(index: int, count: int = 32):
    """The exporter's per-block flags (tools/export_seedvr2_dit_ncnn.py:204-206):
    shared weights from block 10, last layer, odd blocks shifted."""
    return index >= 10, index == count - 1, index % 2 == 1


def write_model_dir(root: Path, input_w, blocks_w, output_w, *, dim, heads, mlp_hidden, video_channels=33,
                    text_channels=5120, output_channels=16, storage="fp16") -> dict:
    """A whole DiT directory in the layout SeedVR2DiT::load reads
    (src/model/dit.cpp:120-174).  Returns the decoded weights."""
    root.mkdir(parents=True, exist_ok=True)
    dec = {"input": write_input_files(root / "seedvr2_dit_input.ncnn.param", root / "seedvr2_dit_input.ncnn.bin",
                                      input_w, dim=dim, video_channels=video_channels,
                                      text_channels=text_channels, storage=storage),
           "output": write_output_files(root / "seedvr2_dit_output.ncnn.param",
                                        root / "seedvr2_dit_output.ncnn.bin", output_w, dim=dim,
                                        output_channels=output_channels, storage=storage),
           "blocks": []}
    for i, w in enumerate(blocks_w):
        shared, last, shifted = block_flags(i, len(blocks_w))
        stem = f"seedvr2_dit_block_{i:02d}.ncnn"
        write_param(root / f"{stem}.param", index=i, shared=shared, last=last, shifted=shifted, dim=dim,
                    heads=heads, mlp_hidden=mlp_hidden)
        dec["blocks"].append(write_bin(root / f"{stem}.bin", w, shared=shared, storage=storage))
    return dec
