"""Pins the oracle's arithmetic (a restatement of the reference CPU layer,
src/layers/seedvr2_dit_block.cpp) against checks that do not retype its
formulas:
  * bf16 rounding (:68-79) against torch's float -> bfloat16 cast over every
    exponent/mantissa-high pattern with tie, near-tie and random low halves;
  * attention (:1045-1079) against textbook softmax(q k^T / sqrt(d)) v in
    float64, written as one global masked attention over all tokens (each
    video query sees its own window's video keys plus every text key; a text
    query's output is the mean over windows), so a wrong window, a dropped
    text key, a transposed operand or a missing scale all fail;
  * special cases: one token (out = v), identical keys (out = mean of v);
  * the q/k prologue (:942-974) against RMSNorm + complex rotation
    e^{i pos freq} in float64 with the reference's positions
    (window-local video (L_txt + t - t0, y - h0, x - w0), text (l, l, l));
  * the elementwise functions (:770-825, :1093-1112) against float64 closed
    forms, and InnerProduct against a float64 matrix product;
  * the block forward (:1114-1267) against a Python composition of the
    oracle's own pieces in the order the reference runs them.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import winplan_exact as wx
from parity import bf16_exact, reference_freqs

HD = 128


# ------------------------------------------------------------------ bf16

def test_bf16_matches_torch_over_all_high_halves(orc):
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFE, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x1234, 0xC0DE, 0x4000],
                    dtype=np.uint32)
    bits = (hi[:, None] | lows[None, :]).ravel()
    x = bits.view(np.float32)
    finite_or_inf = ~np.isnan(x)
    x = x[finite_or_inf]
    got = orc.bf16_array(x)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).float().numpy()
    same = (got.view(np.uint32) == ref.view(np.uint32))
    assert same.all(), f"{int((~same).sum())} mismatches, e.g. {x[~same][:4]}"


def test_bf16_ties_go_to_even(orc):
    # 1 + 2^-8 lies exactly between 1 and 1 + 2^-7: the even neighbour is 1
    assert orc.bf16(1.0 + 2.0 ** -8) == 1.0
    # 1 + 3 * 2^-8 lies between 1 + 2^-7 and 1 + 2^-6: the even one is 1 + 2^-6
    assert orc.bf16(1.0 + 3 * 2.0 ** -8) == 1.0 + 2.0 ** -6
    assert orc.bf16(-(1.0 + 2.0 ** -8)) == -1.0
    assert np.isinf(orc.bf16(np.float32(3.4028235e38)))  # rounds past max bf16 to inf


def test_expf_is_correctly_rounded_and_within_an_ulp_of_libm(orc):
    """orc_expf, the oracle's std::exp(float) (softmax and silu), equals exp
    in float64 rounded once to float32 (closed form), and differs from the host
    libm's expf (the function the reference calls) by at most one ulp."""
    import ctypes
    import ctypes.util
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.uniform(-40.0, 8.0, 20000), [0.0, -0.0, -1e-30, 1e-30, -87.0, 88.0, -104.0]])
    x = x.astype(np.float32)
    lib = orc.load()
    got = np.array([lib.orc_expf(ctypes.c_float(v)) for v in x], dtype=np.float32)
    want = np.exp(x.astype(np.float64)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.expf.argtypes = [ctypes.c_float]
    libm.expf.restype = ctypes.c_float
    host = np.array([libm.expf(ctypes.c_float(v)) for v in x], dtype=np.float32)
    ulps = np.abs(host.view(np.int32).astype(np.int64) - got.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1
    assert (ulps > 0).mean() < 5e-3


# ------------------------------------------------------------------ attention

def _textbook(vid_qkv, txt_qkv, T, H, W, heads, windows, scale=HD ** -0.5):
    """Global masked attention in float64 on bf16-rounded q, k, v (no norm,
    no rotation).  Returns (video outputs [Lv, D], per-window text outputs
    [nW, Lt, D])."""
    D = heads * HD
    Lv, Lt = vid_qkv.shape[0], txt_qkv.shape[0]
    allx = np.concatenate([vid_qkv, txt_qkv]).astype(np.float32)
    allx = bf16_exact(allx).astype(np.float64)
    win_of = np.full(Lv, -1)
    for wi, (t0, t1, h0, h1, w0, w1) in enumerate(windows):
        for t in range(t0, t1):
            for y in range(h0, h1):
                for x in range(w0, w1):
                    win_of[(t * H + y) * W + x] = wi
    vid_out = np.zeros((Lv, D))
    txt_w = np.zeros((len(windows), Lt, D))
    for h in range(heads):
        q = allx[:, h * HD:(h + 1) * HD]
        k = allx[:, D + h * HD:D + (h + 1) * HD]
        v = allx[:, 2 * D + h * HD:2 * D + (h + 1) * HD]
        s = (q @ k.T) * scale
        for wi in range(len(windows)):
            keys = np.concatenate([np.nonzero(win_of == wi)[0], Lv + np.arange(Lt)])
            queries = keys
            ss = s[np.ix_(queries, keys)]
            p = np.exp(ss - ss.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            o = p @ v[keys]
            nv = len(keys) - Lt
            vid_out[keys[:nv], h * HD:(h + 1) * HD] = o[:nv]
            txt_w[wi, :, h * HD:(h + 1) * HD] = o[nv:]
    return vid_out, txt_w


@pytest.mark.parametrize("T,H,W,Lt,heads,shifted,win", [
    (2, 4, 5, 3, 2, False, (1, 2, 3)),
    (2, 4, 5, 3, 2, True, (1, 2, 3)),
    (3, 5, 4, 7, 1, True, (2, 3, 2)),
    (2, 2, 2, 3, 1, True, (0, 0, 0)),
])
def test_attention_matches_global_masked_textbook(orc, T, H, W, Lt, heads, shifted, win):
    rng = np.random.default_rng(T * 100 + H * 10 + W + shifted)
    D = heads * HD
    vid = rng.standard_normal((T * H * W, 3 * D)).astype(np.float32)
    txt = rng.standard_normal((Lt, 3 * D)).astype(np.float32)
    windows = wx.plan(T, H, W, shifted, *win)
    ov, ot, caps = orc.window_attention(vid, txt, T, H, W, heads=heads, qk_norm=False, rope_mode=orc.ROPE_NONE,
                                        shifted=shifted, wt=win[0], wh=win[1], ww=win[2], capture=True)
    ref_v, ref_tw = _textbook(vid, txt, T, H, W, heads, windows)
    # pre-rounding values in window-sequence order
    off = 0
    pre_v = np.zeros_like(ref_v)
    pre_tw = np.zeros_like(ref_tw)
    for wi, (t0, t1, h0, h1, w0, w1) in enumerate(windows):
        rows = [(t * H + y) * W + x for t in range(t0, t1) for y in range(h0, h1) for x in range(w0, w1)]
        pre_v[rows] = caps["pre"][off:off + len(rows)]
        pre_tw[wi] = caps["pre"][off + len(rows):off + len(rows) + Lt]
        off += len(rows) + Lt
    assert np.abs(pre_v - ref_v).max() < 2e-6
    assert np.abs(pre_tw - ref_tw).max() < 2e-6
    # outputs are the bf16 of the pre-rounding values; text averages them
    assert np.array_equal(ov, orc.bf16_array(pre_v.astype(np.float32)))
    acc = np.zeros((Lt, D), np.float32)
    for wi in range(len(windows)):
        acc = acc + orc.bf16_array(pre_tw[wi].astype(np.float32))
    assert np.array_equal(ot, acc * np.float32(np.float32(1) / np.float32(len(windows))))


def test_attention_single_token_returns_v(orc):
    rng = np.random.default_rng(5)
    vid = rng.standard_normal((1, 3 * HD)).astype(np.float32)
    ov, _ = orc.window_attention(vid, np.zeros((0, 3 * HD), np.float32), 1, 1, 1, heads=1, qk_norm=True,
                                 rope_mode=orc.ROPE_REFERENCE, freqs=reference_freqs())
    assert np.array_equal(ov[0], bf16_exact(vid[0, 2 * HD:]))


def test_attention_identical_keys_average_values(orc):
    rng = np.random.default_rng(6)
    n = 12
    vid = rng.standard_normal((n, 3 * HD)).astype(np.float32)
    vid[:, HD:2 * HD] = vid[0, HD:2 * HD]  # every key the same, no rotation: uniform weights
    ov, _ = orc.window_attention(vid, np.zeros((0, 3 * HD), np.float32), 1, 3, 4, heads=1, qk_norm=False,
                                 rope_mode=orc.ROPE_NONE, wt=1, wh=3, ww=4)
    mean = bf16_exact(vid[:, 2 * HD:]).astype(np.float64).mean(axis=0)
    assert np.abs(ov - mean).max() <= np.abs(mean).max() * 2 ** -8 + 1e-7


def test_text_average_single_window_is_identity(orc):
    rng = np.random.default_rng(7)
    vid = rng.standard_normal((2 * 3 * 4, 3 * HD)).astype(np.float32)
    txt = rng.standard_normal((5, 3 * HD)).astype(np.float32)
    _, ot, caps = orc.window_attention(vid, txt, 2, 3, 4, heads=1, rope_mode=orc.ROPE_REFERENCE,
                                       freqs=reference_freqs(), wt=2, wh=3, ww=4, capture=True)
    assert np.array_equal(ot, orc.bf16_array(caps["pre"][24:]))


# ------------------------------------------------------------------ prologue

def _rope_expect(x, gamma, pos, mode, freqs, eps=1e-5):
    """RMSNorm * gamma then complex rotation in float64; angles are the
    float32 products float(pos) * freq the reference forms."""
    y = x.astype(np.float64)
    y = y / np.sqrt((y * y).mean() + eps) * gamma.astype(np.float64)
    if mode == 0:
        layout = [(a * 42, 21, freqs) for a in range(3)]
    else:
        th = [1.0 / 10000.0 ** (np.arange(0, n, 2) / n) for n in (32, 48, 48)]
        layout = [(0, 16, th[0]), (32, 24, th[1]), (80, 24, th[2])]
    out = y.copy()
    for a, (off, npairs, fr) in enumerate(layout):
        for p in range(npairs):
            ang = float(np.float32(np.float32(pos[a]) * np.float32(fr[p])))
            z = complex(y[off + 2 * p], y[off + 2 * p + 1]) * np.exp(1j * ang)
            out[off + 2 * p], out[off + 2 * p + 1] = z.real, z.imag
    return out


@pytest.mark.parametrize("mode", [0, 1])
def test_prologue_is_norm_then_rotation(orc, mode):
    T, H, W, Lt = 3, 5, 6, 4
    rng = np.random.default_rng(11 + mode)
    vid = (rng.standard_normal((T * H * W, 3 * HD)) * 2).astype(np.float32)
    txt = (rng.standard_normal((Lt, 3 * HD)) * 2).astype(np.float32)
    g = rng.uniform(0.5, 1.5, (4, HD)).astype(np.float32)
    freqs = reference_freqs()
    windows = wx.plan(T, H, W, True, 2, 3, 4)
    _, _, caps = orc.window_attention(vid, txt, T, H, W, heads=1, rope_mode=mode, freqs=freqs, gammas=list(g),
                                      shifted=True, wt=2, wh=3, ww=4, capture=True)
    worst = 0.0
    off = 0
    for (t0, t1, h0, h1, w0, w1) in windows:
        seq = [((t * H + y) * W + x, (Lt + t - t0, y - h0, x - w0) if mode == 0 else (t, y, x), True)
               for t in range(t0, t1) for y in range(h0, h1) for x in range(w0, w1)]
        seq += [(l, (l, l, l), False) for l in range(Lt)]
        for s, (row, pos, is_vid) in enumerate(seq):
            src = vid[row] if is_vid else txt[row]
            rotate = is_vid or mode == 0
            for name, col, gam in (("q", 0, g[0] if is_vid else g[2]), ("k", HD, g[1] if is_vid else g[3])):
                e = _rope_expect(src[col:col + HD], gam, pos if rotate else (0, 0, 0), mode, freqs)
                got = caps[name][off + s].astype(np.float64)
                # got is bf16; one bf16 ulp of slack for rounding-boundary cases
                tol = np.abs(e) * 2.0 ** -7 + 1e-6
                assert (np.abs(got - e) <= tol).all(), (name, s, pos)
                worst = max(worst, float(np.abs(got - e).max()))
                # rotation preserves each pair's norm (the unrotated dims 126/127 too)
                n_e = np.hypot(e[0::2], e[1::2])
                n_g = np.hypot(got[0::2], got[1::2])
                assert (np.abs(n_e - n_g) <= n_e * 2.0 ** -7 + 1e-6).all()
            assert np.array_equal(caps["v"][off + s], bf16_exact(src[2 * HD:]))
        off += len(seq)
    assert worst > 0  # the comparison ran on real data


def test_rope_reference_leaves_dims_126_127_unrotated(orc):
    rng = np.random.default_rng(13)
    vid = rng.standard_normal((4, 3 * HD)).astype(np.float32)
    g = np.ones(HD, np.float32)
    _, _, caps = orc.window_attention(vid, np.zeros((0, 3 * HD), np.float32), 1, 2, 2, heads=1,
                                      rope_mode=0, freqs=reference_freqs(), gammas=[g] * 4, wt=1, wh=2, ww=2,
                                      capture=True)

    def normed(row):
        x = vid[row, :HD].astype(np.float32)
        ss = float((x.astype(np.float64) ** 2).sum())
        return x * np.float32(1 / np.sqrt(np.float32(ss / HD) + np.float32(1e-5)))

    # token 3 sits at window-local (0, 1, 1): h and w rotate, 126/127 never do
    assert np.array_equal(caps["q"][3, 126:], bf16_exact(normed(3)[126:]))
    assert not np.array_equal(caps["q"][3, 42:126], bf16_exact(normed(3)[42:126]))
    # token 0 sits at (0, 0, 0) with no text: every angle is zero
    assert np.array_equal(caps["q"][0], bf16_exact(normed(0)))


# ------------------------------------------------------------------ elementwise

@pytest.mark.parametrize("qk_norm", [True, False])
def test_qk_norms_closed_form(orc, qk_norm):
    """orc_qk_norms (the reference's norm_q/k debug captures): per head
    x / sqrt(mean(x^2) + eps) * gamma in float64, before any rotation; the
    identity without the q/k norm; video and text rows take their own gammas."""
    rng = np.random.default_rng(19)
    heads, Lv, Lt = 3, 7, 4
    D = heads * HD
    vid = (rng.standard_normal((Lv, 3 * D)) * 2).astype(np.float32)
    txt = (rng.standard_normal((Lt, 3 * D)) * 2).astype(np.float32)
    gam = [rng.uniform(0.5, 1.5, HD).astype(np.float32) for _ in range(4)]
    out = orc.qk_norms(vid, txt, heads=heads, qk_norm=qk_norm, gammas=gam)
    for o, src, col, g in ((out[0], vid, 0, gam[0]), (out[1], vid, D, gam[1]), (out[2], txt, 0, gam[2]),
                           (out[3], txt, D, gam[3])):
        x = src[:, col:col + D].astype(np.float64).reshape(src.shape[0], heads, HD)
        want = x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + 1e-5) * g if qk_norm else x
        assert np.abs(o.reshape(want.shape) - want).max() <= 1e-6 * max(1.0, np.abs(want).max())


def test_rmsnorm_closed_form(orc):
    rng = np.random.default_rng(20)
    x = (rng.standard_normal((7, 2560)) * 3).astype(np.float32)
    got = orc.rmsnorm_rows(x, 1e-5)
    e = x / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-5)
    assert np.abs(got - e).max() <= 4e-7 * np.abs(e).max()


def test_ada_input_and_residual_closed_forms(orc):
    rng = np.random.default_rng(21)
    D = 256
    x = rng.standard_normal((5, D)).astype(np.float32)
    r = rng.standard_normal((5, D)).astype(np.float32)
    emb = rng.standard_normal(6 * D).astype(np.float32)
    sh, sc, gt = (rng.standard_normal(D).astype(np.float32) for _ in range(3))
    for slot in (0, 3):
        e6 = emb.reshape(D, 6).astype(np.float64)
        got = orc.ada_input(x, emb, sh, sc, slot)
        e = x * (e6[:, slot + 1] + sc) + e6[:, slot] + sh
        assert np.abs(got - e).max() < 1e-5
        got = orc.ada_output_residual(x, r, emb, gt, slot)
        e = x * (e6[:, slot + 2] + gt) + r
        assert np.abs(got - e).max() < 1e-5


def test_swiglu_closed_form(orc):
    rng = np.random.default_rng(22)
    g = (rng.standard_normal(10000) * 4).astype(np.float32)
    v = rng.standard_normal(10000).astype(np.float32)
    got = orc.swiglu(g, v)
    gd = g.astype(np.float64)
    e = gd / (1 + np.exp(-gd)) * v
    assert np.abs(got - e).max() <= 1e-6 * max(1.0, np.abs(e).max())


def test_inner_product_is_wx_plus_b(orc):
    rng = np.random.default_rng(23)
    x = rng.standard_normal((9, 70)).astype(np.float32)
    w = rng.standard_normal((13, 70)).astype(np.float32)
    b = rng.standard_normal(13).astype(np.float32)
    got = orc.inner_product(x, w, b)
    e = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.abs(got - e).max() <= 1e-6 * np.abs(e).max()


# ------------------------------------------------------------------ block

def _rand_branch(rng, D, F):
    def vec(n):
        return (rng.standard_normal(n) * 0.02).astype(np.float32)

    return {
        "attn_shift": vec(D), "attn_scale": vec(D), "attn_gate": vec(D),
        "mlp_shift": vec(D), "mlp_scale": vec(D), "mlp_gate": vec(D),
        "w_qkv": (rng.standard_normal((3 * D, D)) * 0.02).astype(np.float32),
        "w_proj": (rng.standard_normal((D, D)) * 0.02).astype(np.float32), "b_proj": vec(D),
        "norm_q": rng.uniform(0.5, 1.5, HD).astype(np.float32),
        "norm_k": rng.uniform(0.5, 1.5, HD).astype(np.float32),
        "w_gate": (rng.standard_normal((F, D)) * 0.02).astype(np.float32),
        "w_in": (rng.standard_normal((F, D)) * 0.02).astype(np.float32),
        "w_out": (rng.standard_normal((D, F)) * 0.02).astype(np.float32),
    }


def _compose(orc, wts, vid, txt, emb, T, H, W, *, shared, last, shifted, D, heads, eps=1e-5):
    """Appendix of the reference block: the order of seedvr2_dit_block.cpp:1114-1267."""
    vb = wts["vid"]
    tb = vb if shared else wts["txt"]
    xa_v = orc.ada_input(orc.rmsnorm_rows(vid, eps), emb, vb["attn_shift"], vb["attn_scale"], 0)
    xa_t = orc.rmsnorm_rows(txt, eps)
    if not last:
        xa_t = orc.ada_input(xa_t, emb, tb["attn_shift"], tb["attn_scale"], 0)
    qv = orc.inner_product(xa_v, vb["w_qkv"])
    qt = orc.inner_product(xa_t, tb["w_qkv"])
    av, at = orc.window_attention(qv, qt, T, H, W, heads=heads, freqs=wts["freqs"], shifted=shifted,
                                  gammas=[vb["norm_q"], vb["norm_k"], tb["norm_q"], tb["norm_k"]])
    pv = orc.ada_output_residual(orc.inner_product(av, vb["w_proj"], vb["b_proj"]), vid, emb, vb["attn_gate"], 0)
    pt = orc.inner_product(at, tb["w_proj"], tb["b_proj"])
    pt = pt + txt if last else orc.ada_output_residual(pt, txt, emb, tb["attn_gate"], 0)

    def mlp(x, br):
        m = orc.ada_input(orc.rmsnorm_rows(x, eps), emb, br["mlp_shift"], br["mlp_scale"], 3)
        h = orc.swiglu(orc.inner_product(m, br["w_gate"]), orc.inner_product(m, br["w_in"]))
        return orc.ada_output_residual(orc.inner_product(h, br["w_out"]), x, emb, br["mlp_gate"], 3)

    ov = mlp(pv, vb)
    ot = pt * np.float32(2) if last else mlp(pt, tb)
    return ov, ot


@pytest.mark.parametrize("shared,last,shifted", [(False, False, False), (False, False, True),
                                                 (True, True, False), (True, False, True)])
def test_block_forward_is_the_reference_composition(orc, shared, last, shifted):
    rng = np.random.default_rng(30 + 4 * shared + 2 * last + shifted)
    D, heads, F = 256, 2, 384
    T, H, W, Lt = 2, 2, 3, 4
    wts = {"vid": _rand_branch(rng, D, F), "freqs": reference_freqs()}
    if not shared:
        wts["txt"] = _rand_branch(rng, D, F)
    vid = rng.standard_normal((T * H * W, D)).astype(np.float32)
    txt = rng.standard_normal((Lt, D)).astype(np.float32)
    emb = rng.standard_normal(6 * D).astype(np.float32)
    ov, ot = orc.block_forward(wts, vid, txt, emb, T, H, W, dim=D, heads=heads, mlp_hidden=F, shared=shared,
                               last_layer=last, shifted=shifted, wt=1, wh=2, ww=2)
    # the composition runs with the same explicit 1x2x2 windows
    ev, et = _compose_explicit(orc, wts, vid, txt, emb, T, H, W, shared, last, shifted, D, heads)
    assert np.array_equal(ov, ev)
    assert np.array_equal(ot, et)


def _compose_explicit(orc, wts, vid, txt, emb, T, H, W, shared, last, shifted, D, heads):
    orig = orc.window_attention

    def wa(*a, **k):
        k.setdefault("wt", 1)
        k.setdefault("wh", 2)
        k.setdefault("ww", 2)
        return orig(*a, **k)

    orc.window_attention = wa
    try:
        return _compose(orc, wts, vid, txt, emb, T, H, W, shared=shared, last=last, shifted=shifted, D=D,
                        heads=heads)
    finally:
        orc.window_attention = orig


@pytest.mark.parametrize("last", [False, True])
def test_block_stages_compose_to_forward(orc, last):
    """head -> attention -> tail of the oracle equals its block forward bit for
    bit, and the tail's pre-gate projections are proj_out(att) + bias."""
    rng = np.random.default_rng(77 + last)
    D, heads, F = 256, 2, 384
    T, H, W, Lt = 2, 4, 6, 5
    wts = {"vid": _rand_branch(rng, D, F), "txt": _rand_branch(rng, D, F), "freqs": reference_freqs()}
    vid = rng.standard_normal((T * H * W, D)).astype(np.float32)
    txt = rng.standard_normal((Lt, D)).astype(np.float32)
    emb = rng.standard_normal(6 * D).astype(np.float32)
    blk = orc.Block(wts, dim=D, heads=heads, mlp_hidden=F, last_layer=last, shifted=True)
    qv, qt = blk.head(vid, txt, emb)
    av, at = blk.attention(qv, qt, T, H, W)
    vo, to, pv, pt = blk.tail(av, at, vid, txt, emb)
    fv, ft = blk.forward(vid, txt, emb, T, H, W)
    assert np.array_equal(vo, fv) and np.array_equal(to, ft)
    want_pv = av.astype(np.float64) @ wts["vid"]["w_proj"].astype(np.float64).T + wts["vid"]["b_proj"]
    assert np.abs(pv - want_pv).max() < 1e-4
    if last:
        # the last layer's text output is twice (proj + residual)
        want_pt = at.astype(np.float64) @ wts["txt"]["w_proj"].astype(np.float64).T + wts["txt"]["b_proj"]
        assert np.abs(to - 2 * (want_pt + txt)).max() < 1e-4
