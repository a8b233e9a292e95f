"""The DiT at its real size: 1280x720x21 frames (latent 33x6x90x160, patched
grid 6x45x80, 21600 video rows), 32 blocks of width 2560 with 20 heads and a
6912 SwiGLU MLP, 58 text tokens of width 5120, windows 2x9x16 alternating
unshifted / shifted, timestep 1000 (SeedVR2DiT::forward, src/model/dit.cpp:
281-383; the blocks seedvr2_dit_block.cpp:1114-1267).

  * The fp16 DiT: finite, two forwards (the DiT's own workspace, then a
    caller's) bit-identical, and within the reference's full-DiT gate of the
    fp32-compute DiT (NRMSE <= 0.02, cosine >= 0.9998;
    tools/test_seedvr2_dit_ncnn.py:249-250), both DiTs with the same weights
    (fp16 values, N(0, 0.02^2), q/k norm U(0.5, 1.5)) resident on the device.
  * One full-size 720p block in fp32 (the parity mode), unshifted and shifted:
    every stage against the oracle's same stage on the GPU's own stage input,
    on sampled rows (RMSNorm + ada + QKV and proj + MLP work row by row) and
    sampled windows (the attention), at max-abs 2e-3 / mean-abs 2e-4; the
    number of elements that differ from the oracle at all is printed.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import ncnn_files as nf
from parity import reference_freqs

pytestmark = pytest.mark.gpu

T, H, W = 6, 45, 80        # patched grid
WIN = (2, 9, 16)
L_TXT, TEXT_C, LATENT_C, OUT_C = 58, 5120, 33, 16
D, F, HEADS, BLOCKS = 2560, 6912, 20, 32


def metrics(gpu, ref) -> dict:
    g = np.asarray(gpu, np.float64)
    r = np.asarray(ref, np.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    d = g - r
    rms = max(float(np.sqrt(np.mean(r * r))), 1e-12)
    den = max(float(np.sqrt(np.sum(g * g) * np.sum(r * r))), 1e-12)
    return {"finite": bool(np.isfinite(g).all()), "max_abs": float(np.abs(d).max()),
            "mean_abs": float(np.abs(d).mean()), "nrmse": float(np.sqrt(np.mean(d * d))) / rms,
            "cosine": float(np.sum(g * r) / den),
            "differing": int((np.asarray(gpu, np.float32).view(np.uint32)
                              != np.asarray(ref, np.float32).view(np.uint32)).sum())}


@pytest.fixture(scope="module")
def dit_720p():
    """Device weights of the whole DiT (fp16 values), the latent and the text."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(720)

    def randn(shape, std=0.02):
        return (torch.randn(shape, generator=g, device=dev) * std).to(torch.float16).contiguous()

    def unif(shape):
        return (torch.rand(shape, generator=g, device=dev) + 0.5).contiguous()

    blocks, cfgs = [], []
    for i in range(BLOCKS):
        shared, last, shifted = nf.block_flags(i, BLOCKS)
        w = {"freqs": reference_freqs()}
        for br in ("vid",) if shared else ("vid", "txt"):
            w[br] = {f: (unif(s) if f in ("norm_q", "norm_k") else randn(s).float() if f not in nf.MATRICES
                         else randn(s)) for f, s in nf.shapes(D, F).items()}
        blocks.append(w)
        cfgs.append(dict(block_index=i, shared_weights=int(shared), last_layer=int(last),
                         shifted_window=int(shifted), window_t=WIN[0], window_h=WIN[1], window_w=WIN[2]))
    wi = {"w_vid": randn((D, 4 * LATENT_C)), "b_vid": randn((D,)).float(), "w_txt": randn((D, TEXT_C)),
          "b_txt": randn((D,)).float(), "w_time_in": randn((D, 256)).float(), "b_time_in": randn((D,)).float(),
          "w_time_hid": randn((D, D)).float(), "b_time_hid": randn((D,)).float(),
          "w_time_out": randn((6 * D, D)).float(), "b_time_out": randn((6 * D,)).float()}
    wo = {"norm_weight": unif((D,)), "shift": randn((D,)).float(), "scale": randn((D,)).float(),
          "w_proj": randn((4 * OUT_C, D)), "b_proj": randn((4 * OUT_C,)).float()}
    latent = torch.randn((LATENT_C, T, 2 * H, 2 * W), generator=g, device=dev)
    latent[LATENT_C - 1].fill_(1.0)
    text = torch.randn((L_TXT, TEXT_C), generator=g, device=dev)
    return blocks, cfgs, wi, wo, latent, text


def as_f32(w: dict) -> dict:
    return {k: (v.float().contiguous() if isinstance(v, torch.Tensor) else v) for k, v in w.items()}


def build(hip, blocks, cfgs, wi, wo, code):
    conv = (lambda d: d) if code == hip.F16 else as_f32
    inp = hip.DitInput.create(conv(wi), code, on_device=True)
    out = hip.DitOutput.create(conv(wo), code, on_device=True)
    bl = []
    for c, w in zip(cfgs, blocks):
        wd = {k: (conv(v) if isinstance(v, dict) else v) for k, v in w.items()}
        bl.append(hip.DitBlock.from_device(hip.block_config(**c), wd, code))
    return hip.Dit.create(inp, bl, out), (inp, out, bl)


def test_dit_720p_fp16_against_fp32(hip, device, dit_720p):
    blocks, cfgs, wi, wo, latent, text = dit_720p
    out16 = torch.full((OUT_C, T, 2 * H, 2 * W), float("nan"), device=device)
    print("[dit 720p] fp16: own workspace", flush=True)
    dit16, keep16 = build(hip, blocks, cfgs, wi, wo, hip.F16)
    try:
        dit16.forward(latent, text, 1000.0, out16)
        torch.cuda.synchronize()
        a = out16.cpu().numpy()
        print("[dit 720p] fp16: caller workspace", flush=True)
        ws = torch.empty(dit16.workspace_size(T, 2 * H, 2 * W, L_TXT), dtype=torch.uint8, device=device)
        out16.fill_(float("nan"))
        dit16.forward(latent, text, 1000.0, out16, workspace=ws)
        torch.cuda.synchronize()
        b = out16.cpu().numpy()
        del ws
    finally:
        dit16.close()
        for blk in keep16[2]:
            blk.close()
        keep16[0].close()
        keep16[1].close()
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), "own and caller workspace forwards differ"
    print("[dit 720p] fp32 compute (the parity mode)", flush=True)
    dit32, keep32 = build(hip, blocks, cfgs, wi, wo, hip.F32)
    out32 = torch.full_like(out16, float("nan"))
    try:
        dit32.forward(latent, text, 1000.0, out32)
        torch.cuda.synchronize()
        r = out32.cpu().numpy()
    finally:
        dit32.close()
        for blk in keep32[2]:
            blk.close()
        keep32[0].close()
        keep32[1].close()
    rep = metrics(a, r)
    print(f"[dit 720p] fp16 vs fp32: {rep}", flush=True)
    assert np.isfinite(r).all()
    assert rep["nrmse"] <= 0.02 and rep["cosine"] >= 0.9998, rep


@pytest.mark.parametrize("shifted", [False, True], ids=["unshifted", "shifted"])
def test_block_720p_fp32_stages(hip, orc, device, shifted):
    print(f"[block 720p fp32] shifted={shifted}: weights", flush=True)
    rng = np.random.default_rng(7200 + shifted)
    w = nf.random_weights(rng, D, F, shared=False)
    Lv = T * H * W
    vid = rng.standard_normal((Lv, D), dtype=np.float32)
    txt = rng.standard_normal((L_TXT, D), dtype=np.float32)
    emb = rng.standard_normal(6 * D, dtype=np.float32)
    cfg = hip.block_config(shifted_window=int(shifted), window_t=WIN[0], window_h=WIN[1], window_w=WIN[2])
    blk = hip.DitBlock.from_host(cfg, w, hip.F32)
    shapes = {"qkv_vid": (Lv, 3 * D), "qkv_txt": (L_TXT, 3 * D), "attention_vid": (Lv, D),
              "attention_txt": (L_TXT, D), "projected_vid": (Lv, D), "projected_txt": (L_TXT, D),
              "output_vid": (Lv, D), "output_txt": (L_TXT, D)}
    try:
        print(f"[block 720p fp32] shifted={shifted}: forward", flush=True)
        caps = {k: torch.full(s, float("nan"), device=device) for k, s in shapes.items()}
        blk.set_debug(caps)
        blk.set_runtime_shape(T, H, W)
        vo = torch.empty((Lv, D), device=device)
        to = torch.empty((L_TXT, D), device=device)
        blk.forward(torch.from_numpy(vid).to(device), torch.from_numpy(txt).to(device),
                    torch.from_numpy(emb).to(device), vo, to)
        torch.cuda.synchronize()
        g = {k: v.cpu().numpy() for k, v in caps.items()}
        g["vid"], g["txt"] = vo.cpu().numpy(), to.cpu().numpy()
        del caps
    finally:
        blk.set_debug(None)
        blk.close()
    plan = orc.make_windows(T, H, W, shifted, *WIN)
    sample_w = sorted({0, 1, len(plan) // 2, len(plan) - 1})
    win_rows = [((t * H + y) * W + x) for wi in sample_w for (t0, t1, h0, h1, w0, w1) in [plan[wi]]
                for t in range(t0, t1) for y in range(h0, h1) for x in range(w0, w1)]
    rows = np.array(sorted(set(win_rows[::7]) | {0, Lv - 1} | set(rng.integers(0, Lv, 64).tolist())))
    oblk = orc.Block(w, dim=D, heads=HEADS, mlp_hidden=F, shifted=shifted, wt=WIN[0], wh=WIN[1], ww=WIN[2])
    print(f"[block 720p fp32] shifted={shifted}: oracle head on {rows.size} rows", flush=True)
    rq_v, rq_t = oblk.head(vid[rows], txt, emb)
    reps = {"qkv_vid": metrics(g["qkv_vid"][rows], rq_v), "qkv_txt": metrics(g["qkv_txt"], rq_t)}
    print(f"[block 720p fp32] shifted={shifted}: oracle attention on windows {sample_w}", flush=True)
    mask = np.zeros(len(plan), np.uint8)
    mask[sample_w] = 1
    vb, tb = w["vid"], w["txt"]
    ra_v, ra_t = orc.window_attention(
        g["qkv_vid"], g["qkv_txt"], T, H, W, heads=HEADS, freqs=w["freqs"],
        gammas=[vb["norm_q"], vb["norm_k"], tb["norm_q"], tb["norm_k"]], shifted=shifted, wt=WIN[0], wh=WIN[1],
        ww=WIN[2], video_mask=mask)
    reps["attention_vid"] = metrics(g["attention_vid"][win_rows], ra_v[win_rows])
    reps["attention_txt"] = metrics(g["attention_txt"], ra_t)
    print(f"[block 720p fp32] shifted={shifted}: oracle tail on {rows.size} rows", flush=True)
    rv, rt, rp_v, rp_t = oblk.tail(g["attention_vid"][rows], g["attention_txt"], vid[rows], txt, emb)
    reps["projected_vid"] = metrics(g["projected_vid"][rows], rp_v)
    reps["projected_txt"] = metrics(g["projected_txt"], rp_t)
    reps["output_vid"] = metrics(g["vid"][rows], rv)
    reps["output_txt"] = metrics(g["txt"], rt)
    for k, r in reps.items():
        print(f"[block 720p fp32 shifted={shifted}] {k}: max_abs={r['max_abs']:.3g} mean_abs={r['mean_abs']:.3g} "
              f"differing={r['differing']}", flush=True)
    for k, r in reps.items():
        assert r["finite"] and r["max_abs"] <= 2e-3 and r["mean_abs"] <= 2e-4, (k, r)
