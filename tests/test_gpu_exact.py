"""GPU parity of the fp32 parity mode's exact kernels against the oracle, bit
for bit:
  sv2_inner_product_f32   the InnerProduct (seedvr2_dit_block.cpp:27-55): the
                          exact products of each output added in increasing
                          k in double, the bias added in double, one rounding,
                          which is how the oracle evaluates y = W x + b;
  sv2_window_attention    with `exact` set: the reference CPU layer's
                          attention core in its own order and rounding
                          (seedvr2_dit_block.cpp:942-1088).
Both sides evaluate the same float and double operations in the same order,
so the outputs are expected to be identical; a difference can only come from
a double sum or exp landing within 2^-29 of a float rounding boundary, which
the tests allow for a couple of elements per case (and print).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from parity import reference_freqs

pytestmark = pytest.mark.gpu

L_TXT = 58


def differing(a, b) -> int:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    assert a.shape == b.shape
    return int((a.view(np.uint32) != b.view(np.uint32)).sum())


@pytest.mark.parametrize("rows,k,n,bias", [
    (1, 256, 2560, True),        # the time MLP's first product (one row)
    (1, 2560, 15360, True),      # the time MLP's last product (six modulation slots)
    (3, 2560, 2560, False),      # a few rows
    (16, 100, 130, True),        # the most rows of the few-rows form, k and n ragged
    (17, 64, 128, True),         # the fewest rows of the tiled form
    (65, 132, 2560, True),       # vid_in: 4 x 33 latent channels, a ragged row tile
    (130, 2560, 64, True),       # the output head's projection (4 x 16 outputs)
    (300, 2560, 7680, False),    # qkv
    (77, 6912, 2560, False),     # MLP out
    (7, 13, 9, True),            # k and n far from the tiles
])
def test_inner_product_f32_bit_exact(hip, orc, device, rows, k, n, bias):
    print(f"[inner_product_f32] rows={rows} in={k} out={n} bias={bias}", flush=True)
    rng = np.random.default_rng(rows * 7 + k + n)
    x = rng.standard_normal((rows, k), dtype=np.float32)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32) if bias else None
    ref = orc.inner_product(x, w, b)
    y = torch.full((rows, n), float("nan"), device=device)
    hip.inner_product_f32(torch.from_numpy(x).to(device), torch.from_numpy(w).to(device), y,
                          None if b is None else torch.from_numpy(b).to(device))
    torch.cuda.synchronize()
    nd = differing(y.cpu().numpy(), ref)
    print(f"  differing elements: {nd} of {ref.size}", flush=True)
    assert nd <= 2


def exact_case(hip, orc, device, *, T, H, W, Lt, heads, shifted=False, wt=0, wh=0, ww=0, qk_norm=True,
               rope_mode=0, out_dtype="f32", seed=0, video_windows=None):
    print(f"[exact attention] T={T} H={H} W={W} Lt={Lt} heads={heads} shifted={shifted} win=({wt},{wh},{ww}) "
          f"qk_norm={qk_norm} rope={rope_mode} out={out_dtype} seed={seed}", flush=True)
    rng = np.random.default_rng(seed)
    D = heads * 128
    Lv = T * H * W
    vid = rng.standard_normal((Lv, 3 * D), dtype=np.float32)
    txt = rng.standard_normal((Lt, 3 * D), dtype=np.float32)
    gam = rng.uniform(0.5, 1.5, (4, 128)).astype(np.float32) if qk_norm else None
    freqs = reference_freqs()
    plan = orc.make_windows(T, H, W, shifted, wt, wh, ww)
    mask = None
    if video_windows is not None:
        mask = np.zeros(len(plan), np.uint8)
        mask[list(video_windows)] = 1
    ref_v, ref_t, caps = orc.window_attention(
        vid, txt, T, H, W, heads=heads, qk_norm=qk_norm, rope_mode=rope_mode, freqs=freqs,
        gammas=None if gam is None else list(gam), shifted=shifted, wt=wt, wh=wh, ww=ww, capture=True,
        video_mask=mask)
    tdt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[out_dtype]
    attn = hip.WindowAttention(hip.rule(T, H, W, shifted, wt, wh, ww), heads, Lt, qk_norm=qk_norm,
                               rope_mode=rope_mode, freqs=freqs, device=device, exact=True)
    out_v = torch.full((Lv, D), float("nan"), dtype=tdt, device=device)
    out_t = torch.full((Lt, D), float("nan"), dtype=tdt, device=device) if Lt else None
    pre = torch.full(caps["pre"].shape, float("nan"), device=device)
    attn(torch.from_numpy(vid).to(device), torch.from_numpy(txt).to(device) if Lt else None,
         None if gam is None else [torch.from_numpy(g).to(device) for g in gam], out_v, out_t, debug_pre=pre)
    torch.cuda.synchronize()
    gv = out_v.float().cpu().numpy()
    gpre = pre.cpu().numpy()
    seq_rows, vid_rows, off = [], [], 0
    for wi, w in enumerate(plan):
        vl = (w[1] - w[0]) * (w[3] - w[2]) * (w[5] - w[4])
        if mask is None or mask[wi]:
            seq_rows.extend(range(off, off + vl))
            vid_rows.extend(((t * H + y) * W + x) for t in range(w[0], w[1])
                            for y in range(w[2], w[3]) for x in range(w[4], w[5]))
        seq_rows.extend(range(off + vl, off + vl + Lt))
        off += vl + Lt
    ref_cast = torch.from_numpy(ref_v[vid_rows]).to(tdt).float().numpy()
    counts = {"video": differing(gv[vid_rows], ref_cast),
              "pre": differing(gpre[seq_rows], caps["pre"][seq_rows])}
    if Lt:
        gt = out_t.float().cpu().numpy()
        counts["text"] = differing(gt, torch.from_numpy(ref_t).to(tdt).float().numpy())
    print(f"  differing elements: {counts} (video {len(vid_rows) * D}, pre {len(seq_rows) * D})", flush=True)
    assert all(v <= 2 for v in counts.values()), counts


def test_exact_config1_layer(hip, orc, device):
    # grid 2x16x30, 20 heads, 2x8x10 windows, no RoPE, no QK-norm, fp32
    exact_case(hip, orc, device, T=2, H=16, W=30, Lt=L_TXT, heads=20, wt=2, wh=8, ww=10, qk_norm=False,
               rope_mode=2, seed=1)


@pytest.mark.parametrize("shifted", [False, True], ids=["unshifted", "shifted"])
def test_exact_config2_layer(hip, orc, device, shifted):
    exact_case(hip, orc, device, T=2, H=16, W=30, Lt=L_TXT, heads=20, shifted=shifted, wt=2, wh=8, ww=10,
               seed=2 + shifted)


@pytest.mark.parametrize("shifted", [False, True], ids=["unshifted", "shifted"])
def test_exact_reference_adaptive_windows(hip, orc, device, shifted):
    exact_case(hip, orc, device, T=2, H=16, W=30, Lt=L_TXT, heads=4, shifted=shifted, out_dtype="bf16",
               seed=4 + shifted)


@pytest.mark.parametrize("shifted", [False, True], ids=["unshifted", "shifted"])
def test_exact_720p_all_windows(hip, orc, device, shifted):
    # every window of both 720p plans, video and text outputs
    exact_case(hip, orc, device, T=6, H=45, W=80, Lt=L_TXT, heads=20, shifted=shifted, wt=2, wh=9, ww=16,
               seed=10 + shifted, out_dtype="f16")


@pytest.mark.parametrize("case", [
    dict(T=2, H=2, W=2, Lt=3, heads=1, shifted=False),
    dict(T=2, H=2, W=2, Lt=3, heads=1, shifted=True),
    dict(T=1, H=1, W=1, Lt=2, heads=1, shifted=False),
    dict(T=3, H=2, W=2, Lt=4, heads=2, shifted=False),
    dict(T=2, H=5, W=7, Lt=0, heads=2, shifted=True, wt=1, wh=2, ww=3),
    dict(T=3, H=7, W=9, Lt=150, heads=3, shifted=True, wt=2, wh=4, ww=5, rope_mode=1),
])
def test_exact_edge_shapes(hip, orc, device, case):
    exact_case(hip, orc, device, seed=20, **case)


def test_exact_needs_fp32_qkv(hip, device):
    attn = hip.WindowAttention(hip.rule(1, 2, 2, False, 0, 0, 0), 1, 1, device=device, exact=True,
                               freqs=reference_freqs())
    x = torch.zeros((4, 384), dtype=torch.float16, device=device)
    t = torch.zeros((1, 384), dtype=torch.float16, device=device)
    g = [torch.ones(128, device=device) for _ in range(4)]
    with pytest.raises(hip.Sv2Error) as err:
        attn(x, t, g, torch.empty((4, 128), dtype=torch.float16, device=device),
             torch.empty((1, 128), dtype=torch.float16, device=device))
    assert err.value.code == hip.SV2_EINVAL
