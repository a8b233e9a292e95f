"""Pins the oracle's block composition (orc_block_forward, the reference's
SeedVR2DiTBlock::forward, seedvr2_dit_block.cpp:1114-1267) and its DiT chain
(oracle.dit_forward, SeedVR2DiT::forward, src/model/dit.cpp:277-383) against
checks that do not call the oracle's own pieces:

  * a float64 numpy statement of the block written from the model's
    definitions: RMSNorm, the interleaved [dim][6] modulation of the emb blob
    plus the branch vectors, the text branch chosen as the video branch when
    the weights are shared (:1139), per-head q/k RMSNorm * gamma, 3-axis
    rotary embedding as complex rotation, bf16 rounding of q, k, v and of each
    output, softmax(q k^T / sqrt(128)) v per window over the window's video
    tokens and all text tokens (its own window plan, tests/winplan_exact.py),
    text outputs averaged over windows, gated residuals, SwiGLU, and the last
    layer's text rules.  Weights are designed so that a wrong branch, a
    swapped modulation slot or a wrong residual source moves the outputs by
    far more than the gate; that is checked by planting each such mistake in
    the numpy statement and showing the comparison then fails;
  * identities the block's algebra fixes, bit for bit: with W_out = 0 the
    outputs are the gated projections plus the block inputs; with W_proj = 0,
    b_proj = 0 and W_out = 0 they are the inputs themselves (2 x the text
    input on the last layer);
  * one window covering the whole grid: the block's attention is the global
    joint attention of every video and text token;
  * the DiT chain: numpy heads (einops patchify, the sinusoid time MLP, the
    output head) around numpy blocks with the exporter's flags, against the
    oracle's DiT forward.

The numpy statement runs in float64 with bf16 rounding at the reference's
points, the oracle in float32: a value that lands next to a bf16 rounding
boundary may round the other way, so the comparison uses NRMSE <= 1e-3 (a
planted mistake gives 1 and more; the flips give 1e-4 at most here).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import winplan_exact as wx
from parity import reference_freqs

HD = 128
GATE_NRMSE = 1e-3


def bf16(x):
    return torch.from_numpy(np.asarray(x, np.float64).astype(np.float32)).to(torch.bfloat16).double().numpy()


def nrmse(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2)) / max(np.sqrt(np.mean(b * b)), 1e-30))


def rms_norm(x, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def silu(x):
    return x / (1.0 + np.exp(-x))


def rotate(x, pos, freqs):
    """3-axis rotary embedding on adjacent pairs: axis a rotates dims 42a + 2p,
    42a + 2p + 1 (p < 21) by pos[a] * freqs[p]; dims 126, 127 stay."""
    y = x.copy()
    for a in range(3):
        ang = np.outer(pos[:, a], freqs.astype(np.float64))               # [n, 21]
        z = (x[:, 42 * a:42 * a + 42:2] + 1j * x[:, 42 * a + 1:42 * a + 42:2]) * np.exp(1j * ang)
        y[:, 42 * a:42 * a + 42:2] = z.real
        y[:, 42 * a + 1:42 * a + 42:2] = z.imag
    return y


class NpBlock:
    """The block in float64 from the definitions.  `mistake` plants one error
    (for the discrimination checks)."""

    def __init__(self, w, *, dim, heads, eps=1e-5, shared=False, last=False, shifted=False, win=(0, 0, 0),
                 mistake=None):
        self.w, self.D, self.heads, self.eps = w, dim, heads, eps
        self.shared, self.last, self.shifted, self.win = shared, last, shifted, win
        self.mistake = mistake
        self.vb = {k: np.asarray(v, np.float64) for k, v in w["vid"].items()}
        tb = w["vid"] if shared else w["txt"]
        self.tb = {k: np.asarray(v, np.float64) for k, v in tb.items()}
        if mistake == "text_uses_video_branch":
            self.tb = self.vb
        self.freqs = np.asarray(w["freqs"], np.float64)

    def mod(self, emb, br, kind):
        e = np.asarray(emb, np.float64).reshape(self.D, 6)   # emb[c * 6 + slot]
        base = 0 if kind == "attn" else 3
        if self.mistake == "slots_swapped":
            base = 3 - base
        shift = e[:, base] + br[f"{kind}_shift"]
        scale = e[:, base + 1] + br[f"{kind}_scale"]
        gate = e[:, base + 2] + br[f"{kind}_gate"]
        return shift, scale, gate

    def attention(self, qkv_v, qkv_t, T, H, W, windows=None):
        D, Lt = self.D, qkv_t.shape[0]
        windows = windows if windows is not None else wx.plan(T, H, W, self.shifted, *self.win)
        out_v = np.zeros((T * H * W, D))
        out_t = np.zeros((Lt, D))
        for h in range(self.heads):
            cq, ck, cv = h * HD, D + h * HD, 2 * D + h * HD
            acc = np.zeros((Lt, HD))
            for (t0, t1, h0, h1, w0, w1) in windows:
                cells = [(t, y, x) for t in range(t0, t1) for y in range(h0, h1) for x in range(w0, w1)]
                rows = np.array([(t * H + y) * W + x for (t, y, x) in cells], dtype=np.int64)
                pos_v = np.array([(Lt + t - t0, y - h0, x - w0) for (t, y, x) in cells], np.float64).reshape(-1, 3)
                pos_t = np.repeat(np.arange(Lt, dtype=np.float64)[:, None], 3, axis=1)

                def prep(src_v, src_t, c, gv, gt):
                    a = rotate(rms_norm(src_v[rows][:, c:c + HD], self.eps) * gv, pos_v, self.freqs)
                    b = rotate(rms_norm(src_t[:, c:c + HD], self.eps) * gt, pos_t, self.freqs)
                    return bf16(np.concatenate([a, b]))

                q = prep(qkv_v, qkv_t, cq, self.vb["norm_q"], self.tb["norm_q"])
                k = prep(qkv_v, qkv_t, ck, self.vb["norm_k"], self.tb["norm_k"])
                v = bf16(np.concatenate([qkv_v[rows][:, cv:cv + HD], qkv_t[:, cv:cv + HD]]))
                s = q @ k.T / np.sqrt(HD)
                p = np.exp(s - s.max(axis=1, keepdims=True))
                o = bf16((p / p.sum(axis=1, keepdims=True)) @ v)
                out_v[rows, cq:cq + HD] = o[:rows.size]
                acc += o[rows.size:]
            out_t[:, cq:cq + HD] = acc / len(windows)
        return out_v, out_t

    def forward(self, vid, txt, emb, T, H, W, windows=None):
        vid = np.asarray(vid, np.float64)
        txt = np.asarray(txt, np.float64)
        vb, tb = self.vb, self.tb
        sh, sc, g_v = self.mod(emb, vb, "attn")
        xa_v = rms_norm(vid, self.eps) * sc + sh
        sh_t, sc_t, g_t = self.mod(emb, tb, "attn")
        xa_t = rms_norm(txt, self.eps)
        if not self.last:
            xa_t = xa_t * sc_t + sh_t
        att_v, att_t = self.attention(xa_v @ vb["w_qkv"].T, xa_t @ tb["w_qkv"].T, T, H, W, windows)
        res_v = xa_v if self.mistake == "residual_from_normed_input" else vid
        p_v = (att_v @ vb["w_proj"].T + vb["b_proj"]) * g_v + res_v
        p_t = att_t @ tb["w_proj"].T + tb["b_proj"]
        p_t = p_t + txt if self.last else p_t * g_t + txt

        def mlp(x, br):
            msh, msc, mg = self.mod(emb, br, "mlp")
            m = rms_norm(x, self.eps) * msc + msh
            return (silu(m @ br["w_gate"].T) * (m @ br["w_in"].T)) @ br["w_out"].T * mg + x

        return mlp(p_v, vb), (2.0 * p_t if self.last else mlp(p_t, tb))


def designed_branch(rng, D, F, offset):
    """Random weights whose two branches differ in every vector (offset), so
    using one branch for the other changes the result."""
    def vec(n, s=0.1):
        return (rng.standard_normal(n) * s + offset).astype(np.float32)

    return {
        "attn_shift": vec(D), "attn_scale": vec(D), "attn_gate": vec(D),
        "mlp_shift": vec(D), "mlp_scale": vec(D), "mlp_gate": vec(D),
        "w_qkv": (rng.standard_normal((3 * D, D)) * 0.06).astype(np.float32),
        "w_proj": (rng.standard_normal((D, D)) * 0.06).astype(np.float32), "b_proj": vec(D),
        "norm_q": rng.uniform(0.5, 1.5, HD).astype(np.float32),
        "norm_k": rng.uniform(0.5, 1.5, HD).astype(np.float32),
        "w_gate": (rng.standard_normal((F, D)) * 0.06).astype(np.float32),
        "w_in": (rng.standard_normal((F, D)) * 0.06).astype(np.float32),
        "w_out": (rng.standard_normal((D, F)) * 0.06).astype(np.float32),
    }


def designed_emb(rng, D):
    """emb [D][6] with each slot at its own scale, so a swapped slot shows."""
    e = rng.standard_normal((D, 6)) * np.array([0.3, 0.6, 0.9, 1.2, 1.5, 1.8])
    return e.astype(np.float32).reshape(-1)


def case(seed, *, shared, D=256, F=384, T=2, H=4, W=6, Lt=5):
    rng = np.random.default_rng(seed)
    w = {"vid": designed_branch(rng, D, F, 0.0), "freqs": reference_freqs()}
    if not shared:
        w["txt"] = designed_branch(rng, D, F, 0.5)
    vid = rng.standard_normal((T * H * W, D)).astype(np.float32)
    txt = rng.standard_normal((Lt, D)).astype(np.float32)
    return w, vid, txt, designed_emb(rng, D)


VARIANTS = [  # shared, last, shifted, windows
    (False, False, False, (1, 2, 3)),
    (False, False, True, (1, 2, 3)),
    (False, True, True, (2, 2, 2)),
    (True, False, True, (1, 3, 4)),
    (True, True, False, (0, 0, 0)),
]


@pytest.mark.parametrize("shared,last,shifted,win", VARIANTS)
def test_block_matches_numpy_definition(orc, shared, last, shifted, win):
    D, heads, F, T, H, W = 256, 2, 384, 2, 4, 6
    w, vid, txt, emb = case(100 + 8 * shared + 4 * last + 2 * shifted, shared=shared)
    ov, ot = orc.block_forward(w, vid, txt, emb, T, H, W, dim=D, heads=heads, mlp_hidden=F, shared=shared,
                               last_layer=last, shifted=shifted, wt=win[0], wh=win[1], ww=win[2])
    nb = NpBlock(w, dim=D, heads=heads, shared=shared, last=last, shifted=shifted, win=win)
    ev, et = nb.forward(vid, txt, emb, T, H, W)
    rv, rt = nrmse(ov, ev), nrmse(ot, et)
    print(f"[block vs numpy] shared={shared} last={last} shifted={shifted}: nrmse vid {rv:.2e} txt {rt:.2e}")
    assert rv <= GATE_NRMSE and rt <= GATE_NRMSE
    # the gate discriminates: each planted mistake moves an output past it
    mistakes = ["slots_swapped", "residual_from_normed_input"] + ([] if shared else ["text_uses_video_branch"])
    for m in mistakes:
        bv, bt = NpBlock(w, dim=D, heads=heads, shared=shared, last=last, shifted=shifted, win=win,
                         mistake=m).forward(vid, txt, emb, T, H, W)
        worst = max(nrmse(ov, bv), nrmse(ot, bt))
        print(f"  planted {m}: nrmse {worst:.2e}")
        assert worst > 100 * GATE_NRMSE, m


@pytest.mark.parametrize("last", [False, True])
def test_zero_out_projection_leaves_gated_projection(orc, last):
    """W_out = 0: the MLP adds 0 * gate, so the outputs are exactly the gated
    projections plus the block inputs (p_v = proj * (emb_2 + gate) + vid)."""
    D, heads, F, T, H, W = 256, 2, 384, 2, 4, 6
    w, vid, txt, emb = case(200 + last, shared=False)
    for br in ("vid", "txt"):
        w[br]["w_out"] = np.zeros_like(w[br]["w_out"])
    blk = orc.Block(w, dim=D, heads=heads, mlp_hidden=F, last_layer=last, shifted=True)
    ov, ot = blk.forward(vid, txt, emb, T, H, W)
    qv, qt = blk.head(vid, txt, emb)
    av, at = blk.attention(qv, qt, T, H, W)
    _, _, pv, pt = blk.tail(av, at, vid, txt, emb)
    e = emb.reshape(D, 6)
    want_v = pv * (e[:, 2] + w["vid"]["attn_gate"]) + vid
    assert np.array_equal(ov, want_v)
    if last:
        assert np.array_equal(ot, np.float32(2) * (pt + txt))
    else:
        assert np.array_equal(ot, pt * (e[:, 2] + w["txt"]["attn_gate"]) + txt)


@pytest.mark.parametrize("last", [False, True])
def test_zero_projections_return_the_inputs(orc, last):
    """W_proj = 0, b_proj = 0, W_out = 0: both residuals add zero, so the
    block returns its inputs unchanged (the last layer: 2 x the text input)."""
    D, heads, F, T, H, W = 256, 2, 384, 2, 4, 6
    w, vid, txt, emb = case(300 + last, shared=False)
    for br in ("vid", "txt"):
        for f in ("w_proj", "b_proj", "w_out"):
            w[br][f] = np.zeros_like(w[br][f])
    ov, ot = orc.block_forward(w, vid, txt, emb, T, H, W, dim=D, heads=heads, mlp_hidden=F, last_layer=last,
                               shifted=True)
    assert np.array_equal(ov, vid)
    assert np.array_equal(ot, np.float32(2) * txt if last else txt)


def test_single_window_is_global_joint_attention(orc):
    """With one window covering the grid the block's attention is the global
    joint attention of all video and text tokens (positions (L_t + t, y, x))."""
    D, heads, F, T, H, W = 256, 2, 384, 2, 3, 4
    w, vid, txt, emb = case(400, shared=False, T=T, H=H, W=W)
    blk = orc.Block(w, dim=D, heads=heads, mlp_hidden=F, wt=T, wh=H, ww=W)
    qv, qt = blk.head(vid, txt, emb)
    av, at = blk.attention(qv, qt, T, H, W)
    nb = NpBlock(w, dim=D, heads=heads)
    ev, et = nb.attention(qv.astype(np.float64), qt.astype(np.float64), T, H, W,
                          windows=[(0, T, 0, H, 0, W)])
    assert nrmse(av, ev) <= GATE_NRMSE and nrmse(at, et) <= GATE_NRMSE
    # a single window's text average is the window's own text output
    assert np.array_equal(at, bf16(at).astype(np.float32))


def test_dit_chain_matches_numpy_definition(orc):
    """Input head -> blocks (exporter flags) -> output head, numpy against the
    oracle's DiT forward (dit.cpp:277-383)."""
    import ncnn_files as nf
    from test_oracle_heads import _time_mlp_f64, patchify_einops, unpatchify_einops

    rng = np.random.default_rng(500)
    D, heads, F, C, TC, S, OC = 256, 2, 384, 33, 64, 256, 16
    T, Hl, Wl, Lt = 2, 8, 12, 5
    wi = nf.random_input_weights(rng, D, video_channels=C, text_channels=TC, sinusoidal_dim=S, std=0.05)
    wo = nf.random_output_weights(rng, D, output_channels=OC, std=0.05)
    wo["norm_weight"] = rng.uniform(0.5, 1.5, D).astype(np.float32)
    flags = [(False, False, False), (False, False, True), (True, False, False), (True, True, True)]
    weights = []
    for i, (shared, last, shifted) in enumerate(flags):
        w = {"vid": designed_branch(rng, D, F, 0.0), "freqs": reference_freqs()}
        if not shared:
            w["txt"] = designed_branch(rng, D, F, 0.5)
        weights.append(w)
    latent = rng.standard_normal((C, T, Hl, Wl)).astype(np.float32)
    text = rng.standard_normal((Lt, TC)).astype(np.float32)
    oblocks = [orc.Block(w, dim=D, heads=heads, mlp_hidden=F, shared=s, last_layer=l, shifted=sh)
               for w, (s, l, sh) in zip(weights, flags)]
    got = orc.dit_forward(wi, oblocks, wo, latent, text, 1000.0)

    flat = latent.transpose(1, 2, 3, 0).reshape(-1, C).astype(np.float64)
    vid = patchify_einops(flat, T, Hl, Wl, C) @ wi["w_vid"].astype(np.float64).T + wi["b_vid"]
    txt = text.astype(np.float64) @ wi["w_txt"].astype(np.float64).T + wi["b_txt"]
    emb, _ = _time_mlp_f64(wi, 1000.0, S)
    h, w_ = Hl // 2, Wl // 2
    for w, (shared, last, shifted) in zip(weights, flags):
        vid, txt = NpBlock(w, dim=D, heads=heads, shared=shared, last=last, shifted=shifted).forward(
            vid, txt, emb, T, h, w_)
    e = emb.reshape(D, 6)
    normed = rms_norm(vid, 1e-5) * wo["norm_weight"] * (e[:, 1] + wo["scale"]) + e[:, 0] + wo["shift"]
    proj = normed @ wo["w_proj"].astype(np.float64).T + wo["b_proj"]
    want = unpatchify_einops(proj, T, h, w_, OC).reshape(T, Hl, Wl, OC).transpose(3, 0, 1, 2)
    r = nrmse(got, want)
    print(f"[dit chain vs numpy] nrmse {r:.2e}")
    assert got.shape == (OC, T, Hl, Wl) and r <= GATE_NRMSE
