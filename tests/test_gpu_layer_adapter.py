"""The C++ layer boundary on the GPU: tests/cxx/block_runner (built by
build(); the reference runner's command line, tests/dit_block_runner.cpp)
loads exported blocks through SeedVR2DiTBlock_layer_creator and the adapter's
load_param / load_model / create_pipeline and runs forward on host Mats
(sv2_block_forward_host).  It is compared with the same block run through
the device entry points (sv2_block_load + sv2_block_forward +
sv2_block_set_debug) in this process on the same inputs:
  * fp32 (the parity mode, hand-written kernels only): outputs and all 14
    debug captures bit for bit, and the outputs within the block gate of the
    oracle;
  * fp16: the InnerProducts run on hipBLASLt, and a Python process that has
    imported torch resolves libhipblaslt.so.1 to torch's bundled copy while
    the runner loads the ROCm one, so the two may run different kernels for
    a shape.  Each process is reproducible on its own (the kernel choice
    depends on the shape only); across the two, outputs and captures are held
    to the reference's block gate (NRMSE <= 2e-3, cosine >= 0.99999) and the
    number of differing elements is printed.  Cases: the reference runner's synthetic blocks
(tests/dit_block_vulkan_runner.cpp:213-218) and random blocks with text,
shifted, shared/last-layer and fixed-window variants."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

import ncnn_files as nf

pytestmark = pytest.mark.gpu

RUNNER = Path(__file__).resolve().parent / "cxx" / "_build" / "block_runner"
CAPTURES = ("qkv_vid", "qkv_txt", "norm_q_vid", "norm_q_txt", "norm_k_vid", "norm_k_txt", "attention_q",
            "attention_k", "attention_v", "attention_output", "projected_vid", "projected_txt", "output_vid",
            "output_txt")

CASES = [
    # (name, dim, heads, hidden, grid, text, shared, last, shifted, extra params)
    *[(c[-1], c[0], c[1], c[3], c[4:7], c[7], c[8], c[9], c[10], "") for c in nf.RUNNER_CASES],
    ("random_shifted", 256, 2, 512, (3, 8, 12), 7, False, False, True, ""),
    ("random_shared_last", 256, 2, 512, (3, 8, 12), 5, True, True, False, ""),
    ("random_fixed_windows", 256, 2, 512, (3, 8, 12), 6, False, False, True, "9=2 10=4 11=6"),
    ("random_no_text", 256, 2, 512, (2, 6, 10), 0, False, False, False, ""),
]


def read_matrix(path: Path) -> np.ndarray:
    rows, cols = np.fromfile(path, "<i4", 2)
    return np.fromfile(path, "<f4", offset=8).reshape(rows, cols)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_runner_equals_device_entry_points(hip, orc, device, tmp_path, case, dtype):
    name, dim, heads, hidden, (T, H, W), L, shared, last, shifted, extra = case
    assert RUNNER.exists(), "tests/cxx/_build/block_runner is not built (build() compiles it)"
    print(f"[layer adapter] {name} {dtype}", flush=True)
    rng = np.random.default_rng(abs(hash(name)) % 1000)
    if name in [c[-1] for c in nf.RUNNER_CASES]:
        w = nf.runner_weights(dim, 128, hidden, shared)
        vid, txt, emb = nf.runner_inputs(dim, T, H, W, L)
    else:
        w = nf.random_weights(rng, dim, hidden, shared=shared)
        vid = rng.standard_normal((T * H * W, dim), dtype=np.float32)
        txt = rng.standard_normal((L, dim), dtype=np.float32)
        emb = rng.standard_normal(6 * dim, dtype=np.float32)
    param, binf = tmp_path / "b.param", tmp_path / "b.bin"
    nf.write_param(param, shared=shared, last=last, shifted=shifted, dim=dim, heads=heads, mlp_hidden=hidden,
                   extra=extra)
    dec = nf.write_bin(binf, w, shared=shared, storage="fp16")
    files = {k: tmp_path / f"{k}.f32" for k in ("vid", "txt", "emb")}
    for k, a in (("vid", vid), ("txt", txt), ("emb", emb)):
        np.ascontiguousarray(a, "<f4").tofile(files[k])
    env = dict(os.environ, SEEDVR2_FP16="1" if dtype == "f16" else "0")
    cmd = [str(RUNNER), param, binf, files["vid"], T * H * W, files["txt"], L, files["emb"], T, H, W,
           tmp_path / "vo.f32", tmp_path / "to.f32", tmp_path / "cap"]
    r = subprocess.run([str(c) for c in cmd], capture_output=True, text=True, timeout=120, env=env)
    print(r.stdout.strip(), r.stderr.strip(), flush=True)
    assert r.returncode == 0, r.stderr
    rv, rt = read_matrix(tmp_path / "vo.f32"), read_matrix(tmp_path / "to.f32")
    assert rv.shape == (T * H * W, dim) and rt.shape == (L, dim)

    code = hip.F32 if dtype == "f32" else hip.F16
    td = torch.float32 if dtype == "f32" else torch.float16
    blk = hip.DitBlock.load(param, binf, code)
    try:
        cfg = blk.config
        blk.set_runtime_shape(T, H, W)
        S = blk.window_rows(L)
        shapes = {"qkv_vid": (T * H * W, 3 * dim), "qkv_txt": (L, 3 * dim), "attention_q": (S, dim),
                  "attention_k": (S, dim), "attention_v": (S, dim), "attention_output": (S, dim)}
        caps = {k: torch.full(shapes.get(k, (L if k.endswith("txt") else T * H * W, dim)), float("nan"),
                              device=device) for k in CAPTURES}
        blk.set_debug({k: c for k, c in caps.items() if c.numel()})
        v = torch.from_numpy(vid).to(device=device, dtype=td)
        t = torch.from_numpy(txt).to(device=device, dtype=td)
        vo, to = torch.full_like(v, float("nan")), torch.full_like(t, float("nan"))
        blk.forward(v, t if L else None, torch.from_numpy(emb).to(device), vo, to if L else None)
        torch.cuda.synchronize()
        blk.set_debug(None)
        dv, dt = vo.float().cpu().numpy(), to.float().cpu().numpy()
        g = {k: c.cpu().numpy() for k, c in caps.items()}
    finally:
        blk.close()
    pairs = [("vid_out", rv, dv), ("txt_out", rt, dt)]
    for k in CAPTURES:
        c = read_matrix(tmp_path / f"cap_{k}.f32")
        assert c.shape == g[k].shape, (k, c.shape, g[k].shape)
        pairs.append((k, c, g[k]))
    for k, a, b in pairs:
        differing = int((a.view(np.uint32) != b.view(np.uint32)).sum())
        if differing:
            print(f"  {k}: {differing} of {a.size} elements differ", flush=True)
        if dtype == "f32":
            assert differing == 0, k
        elif a.size:
            d = a.astype(np.float64) - b
            rms = max(float(np.sqrt(np.mean(b.astype(np.float64) ** 2))), 1e-12)
            cos = float(np.sum(a * b.astype(np.float64)) /
                        max(np.sqrt(np.sum(a.astype(np.float64) ** 2) * np.sum(b.astype(np.float64) ** 2)), 1e-30))
            assert np.isfinite(a).all() and float(np.sqrt(np.mean(d * d))) / rms <= 2e-3 and cos >= 0.99999, k
    if dtype == "f32":
        ov, ot = orc.block_forward(dec, vid, txt, emb, T, H, W, dim=dim, heads=heads, mlp_hidden=hidden,
                                   eps=cfg.norm_eps, shared=shared, last_layer=last, shifted=shifted,
                                   wt=cfg.window_t, wh=cfg.window_h, ww=cfg.window_w)
        for a, b in ((rv, ov), (rt, ot)):
            if not a.size:
                continue
            d = np.abs(a.astype(np.float64) - b)
            assert d.max() <= 2e-3 and d.mean() <= 2e-4, (d.max(), d.mean())


CHAINS = [
    # blocks as (shared, last, shifted): an unshifted non-shared block, a
    # shifted shared one, then (in the 3-block chain) a shared last layer
    ("two", [(False, False, False), (True, False, True)], 7),
    ("three_last", [(False, False, True), (True, False, False), (True, True, True)], 5),
    ("no_text", [(False, False, False), (False, False, True)], 0),
]


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("chain", CHAINS, ids=[c[0] for c in CHAINS])
def test_device_chain_equals_device_entry_points(hip, device, tmp_path, chain, dtype):
    """The adapter's device forward (sv2::DiTBlockLayer over sv2::DeviceMat
    blobs, enqueue only) chained as the reference DiT chains its blocks on
    VkMat (src/model/dit.cpp:545-581): tests/cxx/block_runner --device-chain
    uploads the inputs once, feeds each block's tops to the next block and
    downloads once.  Against the same blocks chained through sv2_block_forward
    in this process: bit for bit in fp32; within the reference's block gate
    in fp16 (the runner maps the ROCm hipBLASLt, this process torch's copy)."""
    name, flags, L = chain
    assert RUNNER.exists(), "tests/cxx/_build/block_runner is not built (build() compiles it)"
    dim, heads, hidden, (T, H, W) = 256, 2, 512, (3, 8, 12)
    print(f"[device chain] {name} {dtype} blocks={len(flags)} L={L}", flush=True)
    rng = np.random.default_rng(100 + len(flags) + L)
    files = []
    for i, (shared, last, shifted) in enumerate(flags):
        w = nf.random_weights(rng, dim, hidden, shared=shared)
        param, binf = tmp_path / f"b{i}.param", tmp_path / f"b{i}.bin"
        nf.write_param(param, index=i, shared=shared, last=last, shifted=shifted, dim=dim, heads=heads,
                       mlp_hidden=hidden)
        nf.write_bin(binf, w, shared=shared, storage="fp16")
        files += [param, binf]
    vid = rng.standard_normal((T * H * W, dim), dtype=np.float32)
    txt = rng.standard_normal((L, dim), dtype=np.float32)
    emb = rng.standard_normal(6 * dim, dtype=np.float32)
    io = {k: tmp_path / f"{k}.f32" for k in ("vid", "txt", "emb")}
    for k, a in (("vid", vid), ("txt", txt), ("emb", emb)):
        np.ascontiguousarray(a, "<f4").tofile(io[k])
    env = dict(os.environ, SEEDVR2_FP16="1" if dtype == "f16" else "0")
    cmd = [RUNNER, "--device-chain", len(flags), *files, io["vid"], T * H * W, io["txt"], L, io["emb"], T, H, W,
           tmp_path / "vo.f32", tmp_path / "to.f32"]
    r = subprocess.run([str(c) for c in cmd], capture_output=True, text=True, timeout=120, env=env)
    print(r.stdout.strip(), r.stderr.strip(), flush=True)
    assert r.returncode == 0, r.stderr
    rv, rt = read_matrix(tmp_path / "vo.f32"), read_matrix(tmp_path / "to.f32")
    assert rv.shape == (T * H * W, dim) and rt.shape == (L, dim)

    code = hip.F32 if dtype == "f32" else hip.F16
    td = torch.float32 if dtype == "f32" else torch.float16
    v = torch.from_numpy(vid).to(device=device, dtype=td)
    t = torch.from_numpy(txt).to(device=device, dtype=td)
    e = torch.from_numpy(emb).to(device)
    for i in range(len(flags)):
        blk = hip.DitBlock.load(files[2 * i], files[2 * i + 1], code)
        try:
            blk.set_runtime_shape(T, H, W)
            vo, to = torch.full_like(v, float("nan")), torch.full_like(t, float("nan"))
            blk.forward(v, t if L else None, e, vo, to if L else None)
            torch.cuda.synchronize()
        finally:
            blk.close()
        v, t = vo, to
    dv, dt = v.float().cpu().numpy(), t.float().cpu().numpy()
    for k, a, b in (("vid_out", rv, dv), ("txt_out", rt, dt)):
        differing = int((a.view(np.uint32) != b.view(np.uint32)).sum())
        print(f"  {k}: {differing} of {a.size} elements differ", flush=True)
        if dtype == "f32":
            assert differing == 0, k
        elif a.size:
            d = a.astype(np.float64) - b
            rms = max(float(np.sqrt(np.mean(b.astype(np.float64) ** 2))), 1e-12)
            cos = float(np.sum(a * b.astype(np.float64)) /
                        max(np.sqrt(np.sum(a.astype(np.float64) ** 2) * np.sum(b.astype(np.float64) ** 2)), 1e-30))
            assert np.isfinite(a).all() and float(np.sqrt(np.mean(d * d))) / rms <= 2e-3 and cos >= 0.99999, k
