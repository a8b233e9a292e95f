"""GPU parity of the fp16 InnerProduct MFMA kernel (sv2_inner_product_f16,
csrc/gemm.hip), which replaces the block's ncnn InnerProducts
(seedvr2_dit_block.cpp:27-55, :668-674) and fuses the pass after each:
  * plain products against the float64 product of the same fp16 inputs (on
    the CPU, over a sample of rows) rounded to fp16: every element within one
    fp16 ulp of the larger of the two values plus the fp32 accumulation
    allowance 2^-20 * sum_k |x_k w_k| (outputs near zero cancel, and their
    fp32 rounding error is many fp16 ulps of the tiny result; a sequential
    fp32 sum shows the same), and the mean difference far below an ulp;
  * the gated-residual and SwiGLU epilogues against the unfused arithmetic
    (ada_residual / swiglu kernels, seedvr2_dit_block.cpp:807-825,
    :1093-1112) applied in float32 on the host to the kernel's own stored
    products: the residual bit for bit, SwiGLU within one fp16 ulp (the
    host's exp is not the device's);
shapes: the DiT block's products at 720p x 21 frames (21600 rows;
2560 -> 7680, 2560 -> 2560, 2560 -> 2 x 6912, 6912 -> 2560), rows that are
not a multiple of the 256-row tile, one row, and the unsupported shapes'
error codes.

The few-row kernel (sv2_inner_product_f16_few, csrc/gemm_few.hip), which
runs the text branch's products (1-64 rows), is held to the same bars: plain
products against the float64 product of every row, the bias, gated-residual
and SwiGLU epilogues against the unfused arithmetic on its own stored
products, at the text branch's shapes (58 rows; 2560 -> 7680, 2560 -> 2560,
6912 -> 2560 with K split over 2-6 workgroups, 2560 -> 2 x 6912) and at
small and ragged ones; a split product's bits do not depend on what its
workspace held.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def ulp16(x):
    x = np.abs(np.asarray(x, np.float32)).astype(np.float16)
    return np.spacing(np.maximum(x, np.float16(6.1e-5))).astype(np.float32)


def rand16(shape, scale, gen):
    return (torch.randn(shape, generator=gen, device="cuda") * scale).to(torch.float16)


def sample_rows(rows, count=192):
    """The first and last rows, the rows around each 256-row tile edge near
    the end, and a seeded random sample."""
    rng = np.random.default_rng(rows)
    idx = {0, rows - 1, max(0, rows - 257), max(0, rows - 256)}
    idx.update(rng.integers(0, rows, size=min(rows, count)).tolist())
    return np.array(sorted(idx))


def reference64(x, w, idx):
    """float64 product of the fp16 inputs for rows idx rounded to fp16, and
    the fp32 accumulation allowance 2^-20 * sum_k |x_k w_k|."""
    xs = x[torch.from_numpy(idx).cuda()].double().cpu().numpy()
    wd = w.double().cpu().numpy().T
    return (xs @ wd).astype(np.float16), (np.abs(xs) @ np.abs(wd)) * 2.0 ** -20


def assert_ulp(got, ref, ulps=1.0, slack=0.0):
    g = np.asarray(got, np.float32)
    r = np.asarray(ref, np.float32)
    d = np.abs(g - r)
    bad = d > ulps * ulp16(np.maximum(np.abs(g), np.abs(r))) + slack
    assert not bad.any(), f"{int(bad.sum())} of {d.size} beyond {ulps} ulp, max {d.max():.3e}"
    return float(d.mean())


@pytest.mark.parametrize("rows,k,n", [(21600, 2560, 7680), (21600, 6912, 2560), (300, 64, 256), (1, 2560, 512),
                                      (513, 2560, 2560)])
def test_store(hip, rows, k, n):
    gen = torch.Generator(device="cuda").manual_seed(rows + k + n)
    x = rand16((rows, k), 1.0, gen)
    w = rand16((n, k), 0.02, gen)
    y = torch.empty((rows, n), dtype=torch.float16, device="cuda")
    hip.inner_product_f16(x, w, y)
    torch.cuda.synchronize()
    idx = sample_rows(rows)
    got = y.cpu().numpy()[idx]
    ref, slack = reference64(x, w, idx)
    mean = assert_ulp(got, ref, slack=slack)
    assert mean < 2e-4


@pytest.mark.parametrize("rows", [21600, 777])
@pytest.mark.parametrize("bias,gate", [(True, True), (False, True), (True, False)])
def test_residual(hip, rows, bias, gate):
    k, n = 2560, 2560
    gen = torch.Generator(device="cuda").manual_seed(rows + 7)
    x = rand16((rows, k), 1.0, gen)
    w = rand16((n, k), 0.02, gen)
    r = rand16((rows, n), 1.0, gen)
    b = torch.randn(n, generator=gen, device="cuda") * 0.1 if bias else None
    g = torch.randn(n, generator=gen, device="cuda") if gate else None
    p = torch.empty((rows, n), dtype=torch.float16, device="cuda")
    y = torch.empty_like(p)
    hip.inner_product_f16(x, w, p)
    hip.inner_product_f16(x, w, y, hip.EPI_RESIDUAL, bias=b, gate=g, residual=r)
    torch.cuda.synchronize()
    v = p.float().cpu().numpy()
    if bias:
        v = v + b.cpu().numpy()[None, :]
    if gate:
        v = v * g.cpu().numpy()[None, :]
    v = v + r.float().cpu().numpy()
    assert np.array_equal(y.cpu().numpy(), v.astype(np.float16))


@pytest.mark.parametrize("rows,k,f", [(21600, 2560, 6912), (300, 64, 256)])
def test_swiglu(hip, rows, k, f):
    gen = torch.Generator(device="cuda").manual_seed(rows + f)
    x = rand16((rows, k), 1.0, gen)
    wg = rand16((f, k), 0.02, gen)
    wu = rand16((f, k), 0.02, gen)
    pg = torch.empty((rows, f), dtype=torch.float16, device="cuda")
    pu = torch.empty_like(pg)
    y = torch.empty_like(pg)
    hip.inner_product_f16(x, wg, pg)
    hip.inner_product_f16(x, wu, pu)
    hip.inner_product_f16(x, wg, y, hip.EPI_SWIGLU, w_value=wu)
    torch.cuda.synchronize()
    gg = pg.float().cpu().numpy()
    uu = pu.float().cpu().numpy()
    ref = ((gg / (np.float32(1.0) + np.exp(-gg))) * uu).astype(np.float16)
    assert_ulp(y.float().cpu().numpy(), ref)


def test_unsupported_shapes(hip):
    x = torch.zeros((4, 48), dtype=torch.float16, device="cuda")
    w = torch.zeros((256, 48), dtype=torch.float16, device="cuda")
    y = torch.zeros((4, 256), dtype=torch.float16, device="cuda")
    with pytest.raises(hip.Sv2Error) as e:
        hip.inner_product_f16(x, w, y)  # in not a multiple of 64
    assert e.value.code == hip.SV2_EUNSUPPORTED
    x = torch.zeros((4, 64), dtype=torch.float16, device="cuda")
    w = torch.zeros((200, 64), dtype=torch.float16, device="cuda")
    y = torch.zeros((4, 200), dtype=torch.float16, device="cuda")
    with pytest.raises(hip.Sv2Error) as e:
        hip.inner_product_f16(x, w, y)  # out not a multiple of 256
    assert e.value.code == hip.SV2_EUNSUPPORTED


def test_x_operand_just_under_2gib(hip):
    """X of (2^24 - 100) rows x 64 in: 2 GiB less 12.8 KB, the largest kind of
    operand the 32-bit buffer offsets admit, with a ragged last row tile whose
    padded rows' offsets pass INT_MAX (formed unsigned in the kernel, and
    returned as zeros by the buffer resource).  Rows at the start, around the
    2^30-byte and 2^31 - 1 marks and at the end against the float64
    product."""
    rows, k, n = (1 << 24) - 100, 64, 256
    print(f"[gemm] rows={rows} k={k} n={n} (X {rows * k * 2 / 2**30:.4f} GiB)", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(5)
    x = rand16((rows, k), 1.0, gen)
    w = rand16((n, k), 0.02, gen)
    y = torch.empty((rows, n), dtype=torch.float16, device="cuda")
    hip.inner_product_f16(x, w, y)
    torch.cuda.synchronize()
    idx = np.array(sorted({0, 1, (1 << 23) - 1, 1 << 23, rows - 257, rows - 256, rows - 2, rows - 1}))
    got = y[torch.from_numpy(idx).cuda()].cpu().numpy()
    ref, slack = reference64(x, w, idx)
    assert_ulp(got, ref, slack=slack)
    del x, y
    torch.cuda.empty_cache()


# ---- the few-row kernel (sv2_inner_product_f16_few, csrc/gemm_few.hip): the
# text branch's products at 1-64 rows, K split over workgroups with the
# partial sums added in a fixed order

FEW_SHAPES = [(58, 2560, 7680), (58, 6912, 2560), (58, 2560, 2560), (64, 2560, 2560), (1, 2560, 2560),
              (17, 512, 128), (33, 64, 64)]


@pytest.mark.parametrize("rows,k,n", FEW_SHAPES)
def test_few_store(hip, rows, k, n):
    need = hip.load().sv2_inner_product_f16_few_workspace(rows, k, n, hip.EPI_STORE)
    print(f"[few store] rows={rows} k={k} n={n} workspace={need}", flush=True)
    gen = torch.Generator(device="cuda").manual_seed(rows * 7 + k + n)
    x = rand16((rows, k), 1.0, gen)
    w = rand16((n, k), 0.02, gen)
    y = torch.full((rows, n), float("nan"), dtype=torch.float16, device="cuda")
    hip.inner_product_f16_few(x, w, y)
    torch.cuda.synchronize()
    idx = np.arange(rows)
    ref, slack = reference64(x, w, idx)
    mean = assert_ulp(y.cpu().numpy(), ref, slack=slack)
    assert mean < 2e-4
    # the bias form: fp16(fp16(x W^T) + bias), bit for bit on the same sums
    b = torch.randn(n, generator=gen, device="cuda") * 0.1
    yb = torch.empty_like(y)
    hip.inner_product_f16_few(x, w, yb, bias=b)
    torch.cuda.synchronize()
    v = y.float().cpu().numpy() + b.cpu().numpy()[None, :]
    assert np.array_equal(yb.cpu().numpy(), v.astype(np.float16))


@pytest.mark.parametrize("rows,k", [(58, 2560), (58, 6912), (3, 2560)])
@pytest.mark.parametrize("bias,gate", [(True, True), (False, True), (True, False)])
def test_few_residual(hip, rows, k, bias, gate):
    n = 2560
    gen = torch.Generator(device="cuda").manual_seed(rows + k + 3)
    x = rand16((rows, k), 1.0, gen)
    w = rand16((n, k), 0.02, gen)
    r = rand16((rows, n), 1.0, gen)
    b = torch.randn(n, generator=gen, device="cuda") * 0.1 if bias else None
    g = torch.randn(n, generator=gen, device="cuda") if gate else None
    p = torch.empty((rows, n), dtype=torch.float16, device="cuda")
    y = torch.empty_like(p)
    hip.inner_product_f16_few(x, w, p)
    hip.inner_product_f16_few(x, w, y, hip.EPI_RESIDUAL, bias=b, gate=g, residual=r)
    torch.cuda.synchronize()
    v = p.float().cpu().numpy()
    if bias:
        v = v + b.cpu().numpy()[None, :]
    if gate:
        v = v * g.cpu().numpy()[None, :]
    v = v + r.float().cpu().numpy()
    assert np.array_equal(y.cpu().numpy(), v.astype(np.float16))


@pytest.mark.parametrize("rows,k,f", [(58, 2560, 6912), (7, 640, 128), (5, 128, 96)])
def test_few_swiglu(hip, rows, k, f):
    """SwiGLU against the unfused formula on the float64 products rounded to
    fp16.  The fused kernel sums each gate and value product over the whole K
    in one pass (the plain product of the same shape may split K and add in
    another order), so g and u may each sit one fp16 ulp from the float64
    products' roundings: allowed are 3 ulps of the result plus the fp32
    accumulation allowance carried through silu(g) * u (|silu'| < 1.1)."""
    gen = torch.Generator(device="cuda").manual_seed(rows + f + 11)
    x = rand16((rows, k), 1.0, gen)
    wg = rand16((f, k), 0.02, gen)
    wu = rand16((f, k), 0.02, gen)
    y = torch.empty((rows, f), dtype=torch.float16, device="cuda")
    hip.inner_product_f16_few(x, wg, y, hip.EPI_SWIGLU, w_value=wu)
    torch.cuda.synchronize()
    idx = np.arange(rows)
    g16, sg = reference64(x, wg, idx)
    u16, su = reference64(x, wu, idx)
    gg = g16.astype(np.float32)
    uu = u16.astype(np.float32)
    silu = gg / (np.float32(1.0) + np.exp(-gg))
    ref = (silu * uu).astype(np.float16)
    slack = 1.1 * (sg + ulp16(gg)) * np.abs(uu) + (su + ulp16(uu)) * np.abs(silu)
    mean = assert_ulp(y.float().cpu().numpy(), ref, ulps=3.0, slack=slack)
    assert mean < 2e-4


def test_few_split_sums_do_not_depend_on_the_workspace(hip):
    """A split product (58 x 6912 -> 2560: 6 splits) gives the same bits with
    a fresh workspace, with one filled with NaN bytes beforehand, and on a
    repeat: the partial sums are overwritten, then added in a fixed order."""
    rows, k, n = 58, 6912, 2560
    need = hip.load().sv2_inner_product_f16_few_workspace(rows, k, n, hip.EPI_STORE)
    assert need > 0
    gen = torch.Generator(device="cuda").manual_seed(6912)
    x = rand16((rows, k), 1.0, gen)
    w = rand16((n, k), 0.02, gen)
    outs = []
    for fill in (0, 0xFF, 0xFF):
        ws = torch.full((need,), fill, dtype=torch.uint8, device="cuda")
        y = torch.empty((rows, n), dtype=torch.float16, device="cuda")
        hip.inner_product_f16_few(x, w, y, workspace=ws)
        outs.append(y)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    assert bool(torch.isfinite(outs[0]).all())


def test_few_random_shapes(hip):
    """A seeded sweep of few-row shapes (1-64 rows, K 64-4096, N 64-3072, every
    epilogue, K split or not) against the float64 product: store within one
    fp16 ulp plus the accumulation allowance, the residual bit for bit on the
    kernel's own stored product, SwiGLU within 3 ulps plus the carried
    allowance."""
    rng = np.random.default_rng(2024)
    gen = torch.Generator(device="cuda").manual_seed(2024)
    lib = hip.load()
    for case in range(24):
        rows = int(rng.integers(1, 65))
        k = 64 * int(rng.integers(1, 65))
        epi = [hip.EPI_STORE, hip.EPI_RESIDUAL, hip.EPI_SWIGLU][case % 3]
        n = (32 if epi == hip.EPI_SWIGLU else 64) * int(rng.integers(1, 49))
        splits = max(1, lib.sv2_inner_product_f16_few_workspace(rows, k, n, epi) // (rows * n * 4))
        print(f"[few sweep] case {case}: rows={rows} k={k} n={n} epi={epi} splits={splits}", flush=True)
        x = rand16((rows, k), 1.0, gen)
        w = rand16((n, k), 0.02, gen)
        idx = np.arange(rows)
        ref, slack = reference64(x, w, idx)
        y = torch.full((rows, n), float("nan"), dtype=torch.float16, device="cuda")
        if epi == hip.EPI_STORE:
            hip.inner_product_f16_few(x, w, y)
            torch.cuda.synchronize()
            assert_ulp(y.cpu().numpy(), ref, slack=slack)
        elif epi == hip.EPI_RESIDUAL:
            r = rand16((rows, n), 1.0, gen)
            b = torch.randn(n, generator=gen, device="cuda") * 0.1
            g = torch.randn(n, generator=gen, device="cuda")
            p = torch.empty_like(y)
            hip.inner_product_f16_few(x, w, p)
            hip.inner_product_f16_few(x, w, y, hip.EPI_RESIDUAL, bias=b, gate=g, residual=r)
            torch.cuda.synchronize()
            assert_ulp(p.cpu().numpy(), ref, slack=slack)
            v = (p.float().cpu().numpy() + b.cpu().numpy()[None, :]) * g.cpu().numpy()[None, :] + r.float().cpu().numpy()
            assert np.array_equal(y.cpu().numpy(), v.astype(np.float16))
        else:
            wu = rand16((n, k), 0.02, gen)
            hip.inner_product_f16_few(x, w, y, hip.EPI_SWIGLU, w_value=wu)
            torch.cuda.synchronize()
            u16, su = reference64(x, wu, idx)
            gg = ref.astype(np.float32)
            uu = u16.astype(np.float32)
            silu = gg / (np.float32(1.0) + np.exp(-gg))
            sl = 1.1 * (slack + ulp16(gg)) * np.abs(uu) + (su + ulp16(uu)) * np.abs(silu)
            assert_ulp(y.float().cpu().numpy(), (silu * uu).astype(np.float16), ulps=3.0, slack=sl)
