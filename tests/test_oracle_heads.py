"""Pins the oracle's DiT input and output heads (oracle/refcpu.c,
orc_dit_input_forward / orc_dit_output_forward) against independent
formulations, on the CPU:
  * the 1x2x2 patchify and unpatchify permutations (seedvr2_dit_input.cpp:
    336-352, seedvr2_dit_output.cpp:394-413) against einops-style numpy
    reshapes, exposed exactly through identity projections;
  * the timestep sinusoid and time MLP (seedvr2_dit_input.cpp:360-392)
    against a float64 numpy evaluation, and the timestep-0 special case
    (sin = 0, cos = 1);
  * the output head's RMSNorm * weight + ada (seedvr2_dit_output.cpp:368-386)
    against float64 numpy.
"""
from __future__ import annotations

import numpy as np
import pytest

import ncnn_files as nf


def _identity_input(rng, C, dim, text_ch, S):
    w = nf.random_input_weights(rng, dim, video_channels=C, text_channels=text_ch, sinusoidal_dim=S)
    w["w_vid"] = np.eye(dim, 4 * C, dtype=np.float32)
    w["b_vid"] = np.zeros(dim, np.float32)
    w["w_txt"] = np.eye(dim, text_ch, dtype=np.float32)
    w["b_txt"] = np.zeros(dim, np.float32)
    return w


def patchify_einops(video, T, H, W, C):
    h, w = H // 2, W // 2
    v = video.reshape(T, h, 2, w, 2, C)                # t (y dy) (x dx) c
    return v.transpose(0, 1, 3, 2, 4, 5).reshape(T * h * w, 4 * C)  # (t y x) (dy dx c)


def unpatchify_einops(proj, T, h, w, OC):
    p = proj.reshape(T, h, w, 2, 2, OC)                # (t y x) (dy dx c)
    return p.transpose(0, 1, 3, 2, 4, 5).reshape(T * 2 * h * 2 * w, OC)


@pytest.mark.parametrize("T,H,W", [(1, 2, 2), (2, 4, 6), (3, 8, 2)])
def test_patchify_is_the_einops_rearrange(orc, T, H, W):
    rng = np.random.default_rng(T * 100 + H * 10 + W)
    C, text_ch = 2, 8
    dim, S = 4 * C, 8
    w = _identity_input(rng, C, dim, text_ch, S)
    video = rng.standard_normal((T * H * W, C), dtype=np.float32)
    text = rng.standard_normal((3, text_ch), dtype=np.float32)
    vo, to, _ = orc.dit_input_forward(w, video, text, 1.0, T, H, W, sinusoidal_dim=S)
    assert np.array_equal(vo, patchify_einops(video, T, H, W, C))
    assert np.array_equal(to, text)


def test_odd_grid_rejected(orc):
    rng = np.random.default_rng(0)
    w = _identity_input(rng, 2, 8, 8, 8)
    with pytest.raises(RuntimeError):
        orc.dit_input_forward(w, np.zeros((3 * 4, 2), np.float32), np.zeros((1, 8), np.float32), 1.0, 1, 3, 4,
                              sinusoidal_dim=8)


def _time_mlp_f64(w, t, S):
    half = S // 2
    i = np.arange(half, dtype=np.float64)
    f = np.power(10000.0, -i / half)
    s = np.concatenate([np.sin(t * f), np.cos(t * f)])

    def silu(x):
        return x / (1.0 + np.exp(-x))

    h1 = silu(w["w_time_in"].astype(np.float64) @ s + w["b_time_in"])
    h2 = silu(w["w_time_hid"].astype(np.float64) @ h1 + w["b_time_hid"])
    return w["w_time_out"].astype(np.float64) @ h2 + w["b_time_out"], s


@pytest.mark.parametrize("t", [0.0, 1.0, 0.5, 3.0])
def test_time_embedding_matches_float64(orc, t):
    rng = np.random.default_rng(int(t * 10) + 1)
    C, dim, text_ch, S = 2, 16, 8, 32
    w = nf.random_input_weights(rng, dim, video_channels=C, text_channels=text_ch, sinusoidal_dim=S, std=0.3)
    video = rng.standard_normal((4, C), dtype=np.float32)
    _, _, emb = orc.dit_input_forward(w, video, np.zeros((0, text_ch), np.float32), t, 1, 2, 2,
                                      sinusoidal_dim=S)
    want, s = _time_mlp_f64(w, t, S)
    if t == 0.0:
        assert np.array_equal(s[:S // 2], np.zeros(S // 2)) and np.array_equal(s[S // 2:], np.ones(S // 2))
    assert np.allclose(emb, want, rtol=2e-5, atol=2e-6), np.abs(emb - want).max()


def test_sinusoid_halves_not_swapped(orc):
    """With an identity time_in and near-identity layers the first half of the
    embedding follows sin(t f_i) and the second cos(t f_i): swapping them or
    dropping the /half would fail."""
    rng = np.random.default_rng(3)
    dim = S = 8
    w = nf.random_input_weights(rng, dim, video_channels=2, text_channels=8, sinusoidal_dim=S)
    w["w_time_in"] = np.eye(dim, dtype=np.float32)
    w["b_time_in"] = np.zeros(dim, np.float32)
    w["w_time_hid"] = np.eye(dim, dtype=np.float32)
    w["b_time_hid"] = np.zeros(dim, np.float32)
    w["w_time_out"] = np.vstack([np.eye(dim, dtype=np.float32)] * 6)
    w["b_time_out"] = np.zeros(6 * dim, np.float32)
    t = 2.0
    _, _, emb = orc.dit_input_forward(w, np.zeros((4, 2), np.float32), np.zeros((0, 8), np.float32), t, 1, 2, 2,
                                      sinusoidal_dim=S)

    def silu(x):
        return x / (1.0 + np.exp(-x))

    i = np.arange(S // 2)
    s = np.concatenate([np.sin(t * 10000.0 ** (-i / (S // 2))), np.cos(t * 10000.0 ** (-i / (S // 2)))])
    assert np.allclose(emb[:dim], silu(silu(s)), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("T,h,w", [(1, 1, 1), (2, 3, 4)])
def test_output_head_matches_float64_and_einops(orc, T, h, w):
    rng = np.random.default_rng(T + h + w)
    OC = 2
    dim = 4 * OC
    wts = nf.random_output_weights(rng, dim, output_channels=OC, std=0.5)
    wts["w_proj"] = np.eye(4 * OC, dim, dtype=np.float32)
    wts["b_proj"] = np.zeros(4 * OC, np.float32)
    vid = rng.standard_normal((T * h * w, dim), dtype=np.float32) * 2
    emb = rng.standard_normal(6 * dim, dtype=np.float32)
    eps = 1e-5
    out = orc.dit_output_forward(wts, vid, emb, T, h, w, eps=eps)
    x = vid.astype(np.float64)
    inv = 1.0 / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps)
    e = emb.astype(np.float64).reshape(dim, 6)
    normed = x * inv * wts["norm_weight"] * (e[:, 1] + wts["scale"]) + e[:, 0] + wts["shift"]
    want = unpatchify_einops(normed, T, h, w, OC)
    assert out.shape == (T * 4 * h * w, OC)
    assert np.allclose(out, want, rtol=1e-5, atol=1e-5), np.abs(out - want).max()


def test_patchify_unpatchify_roundtrip_layout():
    """The two einops forms used above are inverse permutations."""
    rng = np.random.default_rng(9)
    T, h, w, C = 2, 3, 5, 3
    video = rng.standard_normal((T * 2 * h * 2 * w, C))
    assert np.array_equal(unpatchify_einops(patchify_einops(video, T, 2 * h, 2 * w, C), T, h, w, C), video)
