"""One windowed-attention parity case: seeded inputs, the oracle, the HIP
library through its C ABI, and the parity report (used by the GPU tests and
the smoke check)."""
from __future__ import annotations

import numpy as np

from parity import (assert_parity, assert_text_parity, cast_like, reference_freqs, report,
                    text_report)


def run_attention_case(hip, orc, device, *, T, H, W, Lt, heads, shifted=False, wt=0, wh=0, ww=0, qk_norm=True,
          rope_mode=0, in_dtype="f16", out_dtype="f32", seed=0, video_windows=None):
    import torch
    print(f"[case] T={T} H={H} W={W} Lt={Lt} heads={heads} shifted={shifted} win=({wt},{wh},{ww}) "
          f"qk_norm={qk_norm} rope={rope_mode} in={in_dtype} out={out_dtype} seed={seed}", flush=True)
    rng = np.random.default_rng(seed)
    D = heads * 128
    Lv = T * H * W
    vid = rng.standard_normal((Lv, 3 * D), dtype=np.float32)
    txt = rng.standard_normal((Lt, 3 * D), dtype=np.float32)
    # both sides see the same values: the inputs rounded to the GPU input dtype
    vid, txt = cast_like(vid, in_dtype), cast_like(txt, in_dtype)
    gam = rng.uniform(0.5, 1.5, (4, 128)).astype(np.float32) if qk_norm else None
    freqs = reference_freqs()
    plan = orc.make_windows(T, H, W, shifted, wt, wh, ww)
    mask = None
    if video_windows is not None:
        mask = np.zeros(len(plan), np.uint8)
        mask[list(video_windows)] = 1
    ref_v, ref_t, caps = orc.window_attention(
        vid, txt, T, H, W, heads=heads, qk_norm=qk_norm, rope_mode=rope_mode, freqs=freqs,
        gammas=None if gam is None else list(gam), shifted=shifted, wt=wt, wh=wh, ww=ww,
        capture=True, video_mask=mask)

    tdt = {"f16": torch.float16, "f32": torch.float32, "bf16": torch.bfloat16}
    tv = torch.from_numpy(vid).to(device=device, dtype=tdt[in_dtype])
    tt = torch.from_numpy(txt).to(device=device, dtype=tdt[in_dtype]) if Lt > 0 else None
    gam_t = None if gam is None else [torch.from_numpy(g).to(device) for g in gam]
    attn = hip.WindowAttention(hip.rule(T, H, W, shifted, wt, wh, ww), heads, Lt, eps=1e-5,
                               qk_norm=qk_norm, rope_mode=rope_mode, freqs=freqs, device=device)
    out_v = torch.full((Lv, D), float("nan"), dtype=tdt[out_dtype], device=device)
    out_t = torch.full((Lt, D), float("nan"), dtype=tdt[out_dtype], device=device) if Lt > 0 else None
    pre = torch.full(caps["pre"].shape, float("nan"), dtype=torch.float32, device=device)
    attn(tv, tt, gam_t, out_v, out_t, debug_pre=pre)
    torch.cuda.synchronize()
    gv = out_v.float().cpu().numpy()
    gt = out_t.float().cpu().numpy() if Lt > 0 else np.zeros((0, D), np.float32)
    gpre = pre.cpu().numpy()

    # window-sequence rows that the oracle evaluated, and each window's text rows
    seq_rows = []
    vid_rows = []
    text_rows = []
    off = 0
    for wi, w in enumerate(plan):
        vl = (w[1] - w[0]) * (w[3] - w[2]) * (w[5] - w[4])
        if mask is None or mask[wi]:
            seq_rows.extend(range(off, off + vl))
            vid_rows.extend(((t * H + y) * W + x) for t in range(w[0], w[1])
                            for y in range(w[2], w[3]) for x in range(w[4], w[5]))
        seq_rows.extend(range(off + vl, off + vl + Lt))
        text_rows.append(np.arange(off + vl, off + vl + Lt))
        off += vl + Lt
    vid_rows = np.array(vid_rows, dtype=np.int64)
    seq_rows = np.array(seq_rows, dtype=np.int64)
    text_rows = np.stack(text_rows) if Lt > 0 else np.zeros((len(plan), 0), np.int64)
    rep_v = report(gv[vid_rows], cast_like(ref_v[vid_rows], out_dtype), gpre[seq_rows], caps["pre"][seq_rows])
    rep_t = text_report(gt, ref_t, gpre[text_rows], caps["pre"][text_rows], out_dtype)
    print("video", rep_v, "\ntext", rep_t, flush=True)
    assert_parity(rep_v, "video")
    assert_text_parity(rep_t, "text")
    return rep_v, rep_t
