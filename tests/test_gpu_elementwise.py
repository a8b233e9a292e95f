"""GPU parity of the elementwise kernels around the attention against the CPU
oracle on identical seeded inputs:
  sv2_rmsnorm_ada   apply_rmsnorm + apply_ada_input (seedvr2_dit_block.cpp:770-805)
  sv2_ada_residual  apply_ada_output_and_residual and the last-layer text
                    variants (:807-825, :1198-1209, :1225-1246)
  sv2_swiglu        the SwiGLU gate of apply_mlp (:1093-1112)

Bar: in fp32 every element within 2 fp32 ulps of the oracle (the kernels
follow the reference's operation order without fused multiply-adds; the
per-row sum of squares is a double sum in a different order, and the GPU's
expf differs from glibc's by an ulp); in fp16/bf16 the oracle runs on the
same rounded inputs and the GPU output is within one ulp of the output dtype
of the oracle's fp32 result.  Shapes: a DiT block at 480x256x5 (960 video +
58 text rows, width 2560, MLP hidden 6912), rows that are not a multiple of
the rows a workgroup handles (4, or 16 for launches of 4096 rows and more)
and the widest row the kernel supports.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from parity import cast_like

pytestmark = pytest.mark.gpu

TD = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def ulp_of(x: np.ndarray, dtype: str) -> np.ndarray:
    x = np.abs(np.asarray(x, np.float64))
    mant = {"f32": 24, "f16": 11, "bf16": 8}[dtype]
    tiny = {"f32": 2.0 ** -149, "f16": 2.0 ** -24, "bf16": 2.0 ** -133}[dtype]
    _, e = np.frexp(x)
    return np.maximum(np.ldexp(1.0, e - mant), tiny)


def check(gpu, ref, dtype, ulps):
    gpu = np.asarray(gpu, np.float64)
    ref_r = cast_like(ref, dtype).astype(np.float64)
    assert np.isfinite(gpu).all()
    d = np.abs(gpu - ref_r)
    bound = ulps * ulp_of(np.maximum(np.abs(gpu), np.abs(ref_r)), dtype)
    bad = d > bound
    assert not bad.any(), f"{int(bad.sum())} of {d.size} beyond {ulps} ulp, max diff {d.max():.3e}"
    return float(d.max())


def dev(a, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=TD[dtype])


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("rows,dim", [(1018, 2560), (3, 2560), (5, 4096), (7, 8),
                                      # 16 rows per workgroup (launches of >= 4096 rows,
                                      # every 720p layer) with a ragged last workgroup
                                      (4099, 2560), (4096 + 16 * 3 + 5, 4096)])
@pytest.mark.parametrize("slot,has_ada", [(0, True), (3, True), (0, False)])
def test_rmsnorm_ada(hip, orc, device, dtype, rows, dim, slot, has_ada):
    print(f"[rmsnorm_ada] rows={rows} dim={dim} slot={slot} ada={has_ada} {dtype}", flush=True)
    rng = np.random.default_rng(rows + dim + slot)
    x = cast_like((rng.standard_normal((rows, dim)) * 2).astype(np.float32), dtype)
    emb = rng.standard_normal(6 * dim).astype(np.float32)
    shift = (rng.standard_normal(dim) * 0.02).astype(np.float32)
    scale = (rng.standard_normal(dim) * 0.02).astype(np.float32)
    ref = orc.rmsnorm_rows(x, 1e-5)
    if has_ada:
        ref = orc.ada_input(ref, emb, shift, scale, slot)
    tx = dev(x, dtype, device)
    ty = torch.full_like(tx, float("nan"))
    f32 = lambda a: torch.from_numpy(a).to(device)  # noqa: E731
    hip.rmsnorm_ada(tx, ty, 1e-5, f32(emb), f32(shift), f32(scale), slot, has_ada)
    torch.cuda.synchronize()
    check(ty.float().cpu().numpy(), ref, dtype, 2 if dtype == "f32" else 1)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_ada_residual(hip, orc, device, dtype, mode):
    print(f"[ada_residual] mode={mode} {dtype}", flush=True)
    rows, dim = 1018, 2560
    rng = np.random.default_rng(40 + mode)
    x = cast_like(rng.standard_normal((rows, dim)).astype(np.float32), dtype)
    r = cast_like(rng.standard_normal((rows, dim)).astype(np.float32), dtype)
    emb = rng.standard_normal(6 * dim).astype(np.float32)
    gate = (rng.standard_normal(dim) * 0.02).astype(np.float32)
    slot = 3 if mode == 0 else 0
    if mode == 0:
        ref = orc.ada_output_residual(x, r, emb, gate, slot)
    elif mode == 1:
        ref = x + r
    else:
        ref = x * np.float32(2)
    tx = dev(x, dtype, device)
    tr = dev(r, dtype, device)
    hip.ada_residual(tx, tr, torch.from_numpy(emb).to(device), torch.from_numpy(gate).to(device), slot, mode)
    torch.cuda.synchronize()
    check(tx.float().cpu().numpy(), ref, dtype, 1 if dtype == "f32" else 1)


@pytest.mark.parametrize("rows,dim", [(1, 8), (17, 136), (33, 24), (5, 16384), (3, 16392)],
                         ids=["one-row", "dim136", "dim24", "dim16384", "dim16392-flat"])
def test_ada_residual_gate_shapes(hip, orc, device, rows, dim):
    # mode 0 stages the channel gates in LDS per 16-row workgroup up to dim
    # 16384 (wider rows take the per-element kernel): ragged last workgroups,
    # rows narrower than one pass of the 256 lanes, the largest staged dim
    # and the first unstaged one, all in the oracle's order
    print(f"[ada_residual gate] rows={rows} dim={dim}", flush=True)
    rng = np.random.default_rng(rows * 7 + dim)
    x = cast_like(rng.standard_normal((rows, dim)).astype(np.float32), "f16")
    r = cast_like(rng.standard_normal((rows, dim)).astype(np.float32), "f16")
    emb = rng.standard_normal(6 * dim).astype(np.float32)
    gate = (rng.standard_normal(dim) * 0.02).astype(np.float32)
    ref = orc.ada_output_residual(x, r, emb, gate, 3)
    tx = dev(x, "f16", device)
    tr = dev(r, "f16", device)
    hip.ada_residual(tx, tr, torch.from_numpy(emb).to(device), torch.from_numpy(gate).to(device), 3, 0)
    torch.cuda.synchronize()
    check(tx.float().cpu().numpy(), ref, "f16", 1)


@pytest.mark.parametrize("dtype", ["f32", "f16", "bf16"])
def test_swiglu(hip, orc, device, dtype):
    print(f"[swiglu] {dtype}", flush=True)
    rng = np.random.default_rng(50)
    n = 1018 * 6912
    g = cast_like((rng.standard_normal(n) * 3).astype(np.float32), dtype)
    v = cast_like(rng.standard_normal(n).astype(np.float32), dtype)
    ref = orc.swiglu(g, v)
    tg = dev(g, dtype, device)
    tv = dev(v, dtype, device)
    hip.swiglu(tg, tv)
    torch.cuda.synchronize()
    check(tg.float().cpu().numpy(), ref, dtype, 4 if dtype == "f32" else 1)
