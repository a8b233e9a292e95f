"""Shared helpers of the parity tests: seeded inputs and the comparison report.

The reference rounds every attention output element to bf16
(seedvr2_dit_block.cpp:1074), and at |out| >= 0.25 one bf16 ulp (2^-9 and up)
is already comparable to the 2e-3 max-abs budget.  The GPU path rounds at the
same point, so the two sides differ by more than the budget only where the
pre-rounding values straddle a bf16 rounding boundary.  The report therefore
gives max-abs / mean-abs of the rounded outputs, the count of one-ulp rounding
flips, and max-abs / mean-abs of the pre-rounding values against the oracle's
pre-rounding capture.  The gate:
  * pre-rounding values: max-abs <= 2e-3 and mean-abs <= 2e-4;
  * rounded outputs: mean-abs <= 2e-4, and every element within 2e-3 or a
    single bf16 rounding flip (|diff| <= one bf16 ulp of the larger value).
"""
from __future__ import annotations

import numpy as np

TOL_MAX = 2e-3
TOL_MEAN = 2e-4


def reference_freqs() -> np.ndarray:
    """rope_freqs of SeedVR2-3B: 1/10000^(2i/42), i < 21 (fp32)."""
    i = np.arange(0, 42, 2, dtype=np.float64)
    return (1.0 / (10000.0 ** (i / 42.0))).astype(np.float32)


def fp16_exact(a: np.ndarray) -> np.ndarray:
    """Rounds to fp16-representable values, kept in fp32 for the oracle."""
    return a.astype(np.float16).astype(np.float32)


def bf16_exact(a: np.ndarray) -> np.ndarray:
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).float().numpy()


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """One bf16 ulp at |x| (bf16 keeps 8 significant bits)."""
    x = np.abs(np.asarray(x, dtype=np.float64))
    _, e = np.frexp(x)
    ulp = np.ldexp(1.0, e - 8)
    return np.where(x == 0, np.ldexp(1.0, -133), ulp)


def report(gpu: np.ndarray, ref: np.ndarray, gpu_pre=None, ref_pre=None) -> dict:
    gpu = np.asarray(gpu, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert gpu.shape == ref.shape, (gpu.shape, ref.shape)
    out = {"n": int(gpu.size), "finite": bool(np.isfinite(gpu).all())}
    if gpu.size == 0:
        out.update(max_abs=0.0, mean_abs=0.0, flips=0, flip_frac=0.0, over_tol_not_flip=0)
        return out
    d = np.abs(gpu - ref)
    ulp = bf16_ulp(np.maximum(np.abs(gpu), np.abs(ref)))
    over = d > TOL_MAX
    flip = (d > 0) & (d <= ulp * 1.000001)
    out["max_abs"] = float(d.max())
    out["mean_abs"] = float(d.mean())
    out["flips"] = int(flip.sum())
    out["flip_frac"] = float(flip.mean())
    out["over_tol_not_flip"] = int((over & ~flip).sum())
    if gpu_pre is not None:
        dp = np.abs(np.asarray(gpu_pre, np.float64) - np.asarray(ref_pre, np.float64))
        out["pre_max_abs"] = float(dp.max()) if dp.size else 0.0
        out["pre_mean_abs"] = float(dp.mean()) if dp.size else 0.0
    return out


def cast_like(a: np.ndarray, dtype: str) -> np.ndarray:
    """Rounds fp32 values to an output dtype ("f32", "f16", "bf16"), back in fp32."""
    if dtype == "f16":
        return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_exact(a)
    return np.asarray(a, np.float32)


def window_average(per_window: np.ndarray) -> np.ndarray:
    """The reference's text average (seedvr2_dit_block.cpp:1074-1088): bf16 of
    each window's value, summed in fp32 in window order, times 1/nW."""
    nw = per_window.shape[0]
    acc = np.zeros(per_window.shape[1:], np.float32)
    for w in range(nw):
        acc = acc + bf16_exact(per_window[w])
    return acc * np.float32(np.float32(1.0) / np.float32(nw))


def text_report(gpu_text, ref_text, gpu_pre_w, ref_pre_w, out_dtype: str) -> dict:
    """Text outputs average bf16-rounded per-window values, so a rounding flip
    in window w moves the average by one bf16 ulp of that window's value / nW.
    Reported: the plain diff to the oracle, the flip budget per element (the
    sum over windows of one ulp / nW, from the oracle's own values), and the
    bit-exactness of the GPU reduction against the same average formula
    applied to the GPU's own per-window values."""
    gpu_text = np.asarray(gpu_text, np.float64)
    ref = cast_like(ref_text, out_dtype).astype(np.float64)
    out = {"n": int(gpu_text.size), "finite": bool(np.isfinite(gpu_text).all())}
    if gpu_text.size == 0:
        out.update(max_abs=0.0, mean_abs=0.0, beyond_budget=0, reduce_exact=True)
        return out
    nw = ref_pre_w.shape[0]
    d = np.abs(gpu_text - ref)
    budget = bf16_ulp(ref_pre_w).sum(axis=0) / nw * 1.0001
    if out_dtype != "f32":
        budget = budget + bf16_ulp(ref) if out_dtype == "bf16" else budget + np.abs(ref) * 2.0 ** -10
    out["max_abs"] = float(d.max())
    out["mean_abs"] = float(d.mean())
    out["beyond_budget"] = int(((d > TOL_MAX) & (d > budget)).sum())
    own = cast_like(window_average(gpu_pre_w), out_dtype)
    out["reduce_exact"] = bool(np.array_equal(own.astype(np.float64), gpu_text))
    return out


def assert_text_parity(rep: dict, what: str = "text") -> None:
    assert rep["finite"], f"{what}: non-finite output {rep}"
    assert rep["reduce_exact"], f"{what}: window reduction differs from the reference formula {rep}"
    assert rep["beyond_budget"] == 0, f"{what}: differences beyond 2e-3 and the flip budget {rep}"
    assert rep["mean_abs"] <= TOL_MEAN, f"{what}: mean-abs {rep}"


def assert_parity(rep: dict, what: str = "") -> None:
    assert rep["finite"], f"{what}: non-finite output {rep}"
    assert rep["over_tol_not_flip"] == 0, f"{what}: elements beyond 2e-3 that are not bf16 flips {rep}"
    assert rep["mean_abs"] <= TOL_MEAN, f"{what}: mean-abs {rep}"
    if "pre_max_abs" in rep:
        assert rep["pre_max_abs"] <= TOL_MAX, f"{what}: pre-rounding max-abs {rep}"
        assert rep["pre_mean_abs"] <= TOL_MEAN, f"{what}: pre-rounding mean-abs {rep}"
