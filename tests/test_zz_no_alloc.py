"""sv2_window_attention_no_alloc (the attention on the library's static
scratch, for callers that cannot allocate) against sv2_window_attention with
a caller workspace: the same kernels on the same inputs, so the outputs are
identical bit for bit.  Two calls in a row, the second on a smaller input
(the scratch keeps the first call's contents), then the host-side
rejections: a plan whose scratch exceeds the static array, and the exact
mode."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from parity import reference_freqs

pytestmark = pytest.mark.gpu


def run_both(hip, device, *, T, H, W, Lt, heads, shifted, win, dtype, seed):
    print(f"[no alloc] T={T} H={H} W={W} Lt={Lt} heads={heads} shifted={shifted} win={win} {dtype} seed={seed}",
          flush=True)
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    D = heads * 128
    td = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[dtype]
    vid = torch.randn((T * H * W, 3 * D), generator=g, device=device).to(td)
    txt = torch.randn((Lt, 3 * D), generator=g, device=device).to(td) if Lt else None
    gam = [(torch.rand(128, generator=g, device=device) + 0.5) for _ in range(4)]
    attn = hip.WindowAttention(hip.rule(T, H, W, shifted, *win), heads, Lt, freqs=reference_freqs(), device=device)
    outs = []
    for no_alloc in (False, True):
        ov = torch.full((T * H * W, D), float("nan"), dtype=td, device=device)
        ot = torch.full((Lt, D), float("nan"), dtype=td, device=device) if Lt else None
        if no_alloc:
            attn.run_no_alloc(vid, txt, gam, ov, ot)
        else:
            attn(vid, txt, gam, ov, ot)
        torch.cuda.synchronize()
        outs.append((ov.float().cpu().numpy(), None if ot is None else ot.float().cpu().numpy()))
    (av, at), (bv, bt) = outs
    assert np.isfinite(bv).all()
    assert np.array_equal(av.view(np.uint32), bv.view(np.uint32))
    if Lt:
        assert np.array_equal(at.view(np.uint32), bt.view(np.uint32))


def test_no_alloc_matches_workspace_entry_point_twice(hip, device):
    # the 720p x 21f layer (the largest scratch the array is sized for), then
    # a smaller one that reuses the scratch holding the first call's partials
    run_both(hip, device, T=6, H=45, W=80, Lt=58, heads=20, shifted=True, win=(2, 9, 16), dtype="f16", seed=1)
    run_both(hip, device, T=2, H=16, W=30, Lt=58, heads=20, shifted=False, win=(2, 8, 10), dtype="f16", seed=2)
    run_both(hip, device, T=3, H=7, W=9, Lt=5, heads=3, shifted=True, win=(2, 4, 5), dtype="bf16", seed=3)


def test_no_alloc_rejects_what_the_scratch_cannot_hold(hip, device):
    d = 20 * 128
    vid = torch.zeros((6 * 45 * 80, 3 * d), dtype=torch.float16, device=device)
    gam = [torch.ones(128, device=device) for _ in range(4)]
    # 80 text tokens over 144 windows: 59 MB of partials
    txt = torch.zeros((80, 3 * d), dtype=torch.float16, device=device)
    attn = hip.WindowAttention(hip.rule(6, 45, 80, True, 2, 9, 16), 20, 80, freqs=reference_freqs(), device=device)
    with pytest.raises(hip.Sv2Error) as err:
        attn.run_no_alloc(vid, txt, gam, torch.empty((6 * 45 * 80, d), dtype=torch.float16, device=device),
                          torch.empty((80, d), dtype=torch.float16, device=device))
    assert err.value.code == hip.SV2_EUNSUPPORTED
    exact = hip.WindowAttention(hip.rule(1, 2, 2, False, 0, 0, 0), 1, 1, freqs=reference_freqs(), device=device,
                                exact=True)
    x = torch.zeros((4, 384), device=device)
    with pytest.raises(hip.Sv2Error) as err:
        exact.run_no_alloc(x, torch.zeros((1, 384), device=device), gam, torch.empty((4, 128), device=device),
                           torch.empty((1, 128), device=device))
    assert err.value.code == hip.SV2_EUNSUPPORTED
