"""numpy front end of the CPU oracle (oracle/liborc.so).

TEST INFRASTRUCTURE ONLY: used by tests/, the smoke check and the CPU-baseline
leg of bench.py as the checker.  The product never imports it.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liborc.so"

ROPE_REFERENCE, ROPE_ABSOLUTE, ROPE_NONE = 0, 1, 2

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


class OrcWindow(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("t0", "t1", "h0", "h1", "w0", "w1")]


class OrcAttnCfg(ctypes.Structure):
    _fields_ = [
        ("heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("eps", ctypes.c_float),
        ("qk_norm", ctypes.c_int),
        ("rope_mode", ctypes.c_int),
        ("freqs", ctypes.c_void_p),
        ("rope_theta", ctypes.c_float),
        ("gq_vid", ctypes.c_void_p),
        ("gk_vid", ctypes.c_void_p),
        ("gq_txt", ctypes.c_void_p),
        ("gk_txt", ctypes.c_void_p),
        ("shifted", ctypes.c_int),
        ("wt", ctypes.c_int),
        ("wh", ctypes.c_int),
        ("ww", ctypes.c_int),
        ("threads", ctypes.c_int),
    ]


class OrcBranch(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate",
        "w_qkv", "w_proj", "b_proj", "norm_q", "norm_k", "w_gate", "w_in", "w_out")]


class OrcBlock(ctypes.Structure):
    _fields_ = [
        ("dim", ctypes.c_int), ("heads", ctypes.c_int), ("head_dim", ctypes.c_int),
        ("mlp_hidden", ctypes.c_int), ("eps", ctypes.c_float),
        ("shared", ctypes.c_int), ("last_layer", ctypes.c_int), ("shifted", ctypes.c_int),
        ("wt", ctypes.c_int), ("wh", ctypes.c_int), ("ww", ctypes.c_int),
        ("rope_mode", ctypes.c_int), ("rope_theta", ctypes.c_float), ("qk_norm", ctypes.c_int),
        ("vid", OrcBranch), ("txt", OrcBranch), ("freqs", ctypes.c_void_p), ("threads", ctypes.c_int),
    ]


class OrcDitInput(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("dim", "video_channels", "text_channels", "sinusoidal_dim",
                                            "embedding_dim")] + \
               [(n, ctypes.c_void_p) for n in ("w_vid", "b_vid", "w_txt", "b_txt", "w_tin", "b_tin", "w_thid",
                                               "b_thid", "w_tout", "b_tout")] + [("threads", ctypes.c_int)]


class OrcDitOutput(ctypes.Structure):
    _fields_ = [("dim", ctypes.c_int), ("output_channels", ctypes.c_int), ("eps", ctypes.c_float)] + \
               [(n, ctypes.c_void_p) for n in ("norm", "shift", "scale", "w_proj", "b_proj")] + \
               [("threads", ctypes.c_int)]


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    vp, i = ctypes.c_void_p, ctypes.c_int
    lib.orc_bf16.argtypes = [ctypes.c_float]
    lib.orc_bf16.restype = ctypes.c_float
    lib.orc_expf.argtypes = [ctypes.c_float]
    lib.orc_expf.restype = ctypes.c_float
    lib.orc_bf16_array.argtypes = [vp, vp, ctypes.c_int64]
    lib.orc_adaptive_window.argtypes = [i, i, i, vp, vp, vp]
    lib.orc_make_windows.argtypes = [i, i, i, i, i, i, i, vp, i]
    lib.orc_make_windows.restype = i
    lib.orc_window_attention.argtypes = [ctypes.POINTER(OrcAttnCfg), i, i, i, i, vp, vp, vp, vp,
                                         vp, vp, vp, vp, vp]
    lib.orc_window_attention.restype = i
    lib.orc_qk_norms.argtypes = [ctypes.POINTER(OrcAttnCfg), i, i, vp, vp, vp, vp, vp, vp]
    lib.orc_qk_norms.restype = i
    lib.orc_rmsnorm_rows.argtypes = [vp, i, i, ctypes.c_float]
    lib.orc_ada_input.argtypes = [vp, i, i, vp, vp, vp, i]
    lib.orc_ada_output_residual.argtypes = [vp, vp, i, i, vp, vp, i]
    lib.orc_swiglu.argtypes = [vp, vp, ctypes.c_int64]
    lib.orc_inner_product.argtypes = [vp, i, i, vp, vp, i, vp, i]
    lib.orc_block_forward.argtypes = [ctypes.POINTER(OrcBlock), vp, i, vp, i, vp, i, i, i, vp, vp]
    lib.orc_block_forward.restype = i
    lib.orc_block_head.argtypes = [ctypes.POINTER(OrcBlock), vp, i, vp, i, vp, vp, vp]
    lib.orc_block_head.restype = i
    lib.orc_block_attention.argtypes = [ctypes.POINTER(OrcBlock), i, i, i, i, vp, vp, vp, vp]
    lib.orc_block_attention.restype = i
    lib.orc_block_tail.argtypes = [ctypes.POINTER(OrcBlock), vp, i, vp, i, vp, vp, vp, vp, vp, vp, vp]
    lib.orc_block_tail.restype = i
    lib.orc_dit_input_forward.argtypes = [ctypes.POINTER(OrcDitInput), vp, vp, i, ctypes.c_float, i, i, i,
                                          vp, vp, vp]
    lib.orc_dit_input_forward.restype = i
    lib.orc_dit_output_forward.argtypes = [ctypes.POINTER(OrcDitOutput), vp, vp, i, i, i, vp]
    lib.orc_dit_output_forward.restype = i
    i64, f = ctypes.c_int64, ctypes.c_float
    lib.orc_euler_timesteps.argtypes = [i, vp]
    lib.orc_euler_timesteps.restype = i
    lib.orc_condition_ratio.argtypes = [f, i, i, i]
    lib.orc_condition_ratio.restype = f
    lib.orc_make_condition.argtypes = [vp, vp, vp, i64, f]
    lib.orc_make_dit_input.argtypes = [vp, vp, vp, i64, i]
    lib.orc_standard_deviation.argtypes = [vp, i64]
    lib.orc_standard_deviation.restype = ctypes.c_double
    lib.orc_apply_cfg.argtypes = [vp, vp, vp, i64, f, f]
    lib.orc_euler_step.argtypes = [vp, vp, vp, i64, f, f]
    lib.orc_euler_endpoint.argtypes = [vp, vp, vp, i64, f]
    _lib = lib
    return lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    return None if a is None else a.ctypes.data


def bf16(x: float) -> float:
    return load().orc_bf16(ctypes.c_float(x))


def expf(x: float) -> float:
    """The oracle's std::exp of a float (correctly rounded)."""
    return load().orc_expf(ctypes.c_float(x))


def bf16_array(x):
    x = _f32(x)
    out = np.empty_like(x)
    load().orc_bf16_array(_p(x), _p(out), x.size)
    return out


def adaptive_window(T, H, W):
    out = (ctypes.c_int * 3)()
    load().orc_adaptive_window(T, H, W, ctypes.byref(out, 0), ctypes.byref(out, 4), ctypes.byref(out, 8))
    return tuple(out)


def make_windows(T, H, W, shifted=False, wt=0, wh=0, ww=0):
    lib = load()
    n = lib.orc_make_windows(T, H, W, int(bool(shifted)), wt, wh, ww, None, 0)
    arr = (OrcWindow * max(n, 1))()
    lib.orc_make_windows(T, H, W, int(bool(shifted)), wt, wh, ww, arr, n)
    return [(w.t0, w.t1, w.h0, w.h1, w.w0, w.w1) for w in arr[:n]]


def window_attention(vid_qkv, txt_qkv, T, H, W, *, heads, head_dim=128, eps=1e-5, qk_norm=True,
                     rope_mode=ROPE_REFERENCE, freqs=None, theta=10000.0, gammas=None,
                     shifted=False, wt=0, wh=0, ww=0, threads=0, capture=False, video_mask=None):
    """Returns (vid_out, txt_out) or, with capture=True, also a dict with the
    q/k/v after the prologue and the pre-rounding outputs in window-sequence order."""
    lib = load()
    vid_qkv = _f32(vid_qkv)
    txt_qkv = _f32(txt_qkv)
    D = heads * head_dim
    Lv, Lt = vid_qkv.shape[0], txt_qkv.shape[0]
    assert vid_qkv.shape[1] == 3 * D and (Lt == 0 or txt_qkv.shape[1] == 3 * D)
    assert Lv == T * H * W
    ones = np.ones(head_dim, dtype=np.float32)
    gq_v, gk_v, gq_t, gk_t = [(_f32(g) if g is not None else ones) for g in (gammas or (None,) * 4)]
    fr = _f32(freqs) if freqs is not None else np.zeros(21, dtype=np.float32)
    cfg = OrcAttnCfg(heads, head_dim, eps, int(bool(qk_norm)), rope_mode, _p(fr), theta,
                     _p(gq_v), _p(gk_v), _p(gq_t), _p(gk_t), int(bool(shifted)), wt, wh, ww, threads)
    vid_out = np.zeros((Lv, D), dtype=np.float32)
    txt_out = np.zeros((Lt, D), dtype=np.float32)
    caps = None
    cap_ptrs = [None] * 4
    if capture:
        wins = make_windows(T, H, W, shifted, wt, wh, ww)
        total = sum((w[1] - w[0]) * (w[3] - w[2]) * (w[5] - w[4]) + Lt for w in wins)
        caps = {k: np.zeros((total, D), dtype=np.float32) for k in ("q", "k", "v", "pre")}
        cap_ptrs = [_p(caps[k]) for k in ("q", "k", "v", "pre")]
    mask = None
    if video_mask is not None:
        mask = np.ascontiguousarray(video_mask, dtype=np.uint8)
    rc = lib.orc_window_attention(ctypes.byref(cfg), T, H, W, Lt, _p(vid_qkv), _p(txt_qkv),
                                  _p(vid_out), _p(txt_out), *cap_ptrs, _p(mask))
    if rc != 0:
        raise RuntimeError(f"orc_window_attention failed: {rc}")
    if capture:
        return vid_out, txt_out, caps
    return vid_out, txt_out


def qk_norms(vid_qkv, txt_qkv, *, heads, head_dim=128, eps=1e-5, qk_norm=True, gammas=None):
    """q and k after RMSNorm * gamma, before RoPE (the reference's norm_q/k_vid
    and norm_q/k_txt captures).  Returns (nq_vid, nk_vid, nq_txt, nk_txt)."""
    vid_qkv, txt_qkv = _f32(vid_qkv), _f32(txt_qkv)
    D = heads * head_dim
    ones = np.ones(head_dim, dtype=np.float32)
    g = [(_f32(x) if x is not None else ones) for x in (gammas or (None,) * 4)]
    fr = np.zeros(21, dtype=np.float32)
    cfg = OrcAttnCfg(heads, head_dim, eps, int(bool(qk_norm)), ROPE_NONE, _p(fr), 10000.0,
                     _p(g[0]), _p(g[1]), _p(g[2]), _p(g[3]), 0, 0, 0, 0, 0)
    Lv, Lt = vid_qkv.shape[0], txt_qkv.shape[0]
    out = [np.zeros((Lv, D), np.float32), np.zeros((Lv, D), np.float32), np.zeros((Lt, D), np.float32),
           np.zeros((Lt, D), np.float32)]
    rc = load().orc_qk_norms(ctypes.byref(cfg), Lv, Lt, _p(vid_qkv), _p(txt_qkv), *[_p(o) for o in out])
    if rc != 0:
        raise RuntimeError(f"orc_qk_norms failed: {rc}")
    return tuple(out)


def rmsnorm_rows(x, eps):
    x = _f32(x).copy()
    load().orc_rmsnorm_rows(_p(x), x.shape[0], x.shape[1], eps)
    return x


def ada_input(x, emb, shift, scale, slot_base):
    x = _f32(x).copy()
    emb, shift, scale = _f32(emb), _f32(shift), _f32(scale)
    load().orc_ada_input(_p(x), x.shape[0], x.shape[1], _p(emb), _p(shift), _p(scale), slot_base)
    return x


def ada_output_residual(x, residual, emb, gate, slot_base):
    x = _f32(x).copy()
    residual, emb, gate = _f32(residual), _f32(emb), _f32(gate)
    load().orc_ada_output_residual(_p(x), _p(residual), x.shape[0], x.shape[1], _p(emb), _p(gate), slot_base)
    return x


def swiglu(gate, value):
    g = _f32(gate).copy()
    v = _f32(value)
    load().orc_swiglu(_p(g), _p(v), g.size)
    return g


def inner_product(x, weight, bias=None, threads=0):
    x, weight = _f32(x), _f32(weight)
    b = None if bias is None else _f32(bias)
    rows, n_in = x.shape
    n_out = weight.shape[0]
    y = np.zeros((rows, n_out), dtype=np.float32)
    load().orc_inner_product(_p(x), rows, n_in, _p(weight), _p(b), n_out, _p(y), threads)
    return y


BRANCH_FIELDS = ("attn_shift", "attn_scale", "attn_gate", "mlp_shift", "mlp_scale", "mlp_gate",
                 "w_qkv", "w_proj", "b_proj", "norm_q", "norm_k", "w_gate", "w_in", "w_out")


class Block:
    """One block's parameters and weights for the oracle's block functions.
    weights: {"vid": {field: array}, "txt": {...} (unless shared), "freqs": [21]}."""

    def __init__(self, weights, *, dim, heads, head_dim=128, mlp_hidden, eps=1e-5, shared=False,
                 last_layer=False, shifted=False, wt=0, wh=0, ww=0, rope_mode=ROPE_REFERENCE, theta=10000.0,
                 qk_norm=True, threads=0):
        self._keep = []

        def branch(d):
            arrs = {k: _f32(d[k]) for k in BRANCH_FIELDS}
            self._keep.append(arrs)
            return OrcBranch(*[_p(arrs[k]) for k in BRANCH_FIELDS])

        vb = branch(weights["vid"])
        tb = vb if shared else branch(weights["txt"])
        freqs = _f32(weights["freqs"])
        self._keep.append(freqs)
        self.dim = dim
        self.s = OrcBlock(dim, heads, head_dim, mlp_hidden, eps, int(shared), int(last_layer), int(shifted),
                          wt, wh, ww, rope_mode, theta, int(qk_norm), vb, tb, _p(freqs), threads)

    def forward(self, vid, txt, emb, T, H, W):
        vid, txt, emb = _f32(vid), _f32(txt), _f32(emb)
        vid_out = np.zeros_like(vid)
        txt_out = np.zeros_like(txt)
        rc = load().orc_block_forward(ctypes.byref(self.s), _p(vid), vid.shape[0], _p(txt), txt.shape[0],
                                      _p(emb), T, H, W, _p(vid_out), _p(txt_out))
        if rc != 0:
            raise RuntimeError(f"orc_block_forward failed: {rc}")
        return vid_out, txt_out

    def head(self, vid, txt, emb):
        """qkv of both streams (seedvr2_dit_block.cpp:1141-1156)."""
        vid, txt, emb = _f32(vid), _f32(txt), _f32(emb)
        qv = np.zeros((vid.shape[0], 3 * self.dim), np.float32)
        qt = np.zeros((txt.shape[0], 3 * self.dim), np.float32)
        rc = load().orc_block_head(ctypes.byref(self.s), _p(vid), vid.shape[0], _p(txt), txt.shape[0], _p(emb),
                                   _p(qv), _p(qt))
        if rc != 0:
            raise RuntimeError(f"orc_block_head failed: {rc}")
        return qv, qt

    def attention(self, qkv_v, qkv_t, T, H, W):
        qkv_v, qkv_t = _f32(qkv_v), _f32(qkv_t)
        av = np.zeros((qkv_v.shape[0], self.dim), np.float32)
        at = np.zeros((qkv_t.shape[0], self.dim), np.float32)
        rc = load().orc_block_attention(ctypes.byref(self.s), T, H, W, qkv_t.shape[0], _p(qkv_v), _p(qkv_t),
                                        _p(av), _p(at))
        if rc != 0:
            raise RuntimeError(f"orc_block_attention failed: {rc}")
        return av, at

    def tail(self, att_v, att_t, vid, txt, emb):
        """Outputs and the pre-gate projections from given attention outputs
        (seedvr2_dit_block.cpp:1180-1260)."""
        att_v, att_t, vid, txt, emb = map(_f32, (att_v, att_t, vid, txt, emb))
        vo, to = np.zeros_like(vid), np.zeros_like(txt)
        pv, pt = np.zeros_like(vid), np.zeros_like(txt)
        rc = load().orc_block_tail(ctypes.byref(self.s), _p(att_v), att_v.shape[0], _p(att_t), att_t.shape[0],
                                   _p(vid), _p(txt), _p(emb), _p(vo), _p(to), _p(pv), _p(pt))
        if rc != 0:
            raise RuntimeError(f"orc_block_tail failed: {rc}")
        return vo, to, pv, pt


def block_forward(weights, vid, txt, emb, T, H, W, *, dim, heads, head_dim=128, mlp_hidden,
                  eps=1e-5, shared=False, last_layer=False, shifted=False, wt=0, wh=0, ww=0,
                  rope_mode=ROPE_REFERENCE, theta=10000.0, qk_norm=True, threads=0):
    """weights: {"vid": {field: array}, "txt": {...} (unless shared), "freqs": [21]}."""
    blk = Block(weights, dim=dim, heads=heads, head_dim=head_dim, mlp_hidden=mlp_hidden, eps=eps, shared=shared,
                last_layer=last_layer, shifted=shifted, wt=wt, wh=wh, ww=ww, rope_mode=rope_mode, theta=theta,
                qk_norm=qk_norm, threads=threads)
    return blk.forward(vid, txt, emb, T, H, W)


INPUT_FIELDS = ("w_vid", "b_vid", "w_txt", "b_txt", "w_time_in", "b_time_in", "w_time_hid", "b_time_hid",
                "w_time_out", "b_time_out")
OUTPUT_FIELDS = ("norm_weight", "shift", "scale", "w_proj", "b_proj")


def dit_input_forward(weights, video, text, timestep, T, H, W, *, sinusoidal_dim=256, threads=0):
    """The DiT input head.  weights: {field: array} of INPUT_FIELDS; video
    [T*H*W, C] token-major fp32, text [L, text_channels].  Returns
    (vid_out [T*(H/2)*(W/2), dim], txt_out [L, dim], emb [6*dim])."""
    arrs = {k: _f32(weights[k]) for k in INPUT_FIELDS}
    dim = arrs["b_vid"].shape[0]
    video, text = _f32(video), _f32(text)
    C, tc = video.shape[1], arrs["w_txt"].shape[1]
    cfg = OrcDitInput(dim, C, tc, sinusoidal_dim, arrs["b_time_out"].shape[0],
                      *[_p(arrs[k]) for k in INPUT_FIELDS], threads)
    rows = T * (H // 2) * (W // 2)
    vo = np.zeros((rows, dim), np.float32)
    to = np.zeros((text.shape[0], dim), np.float32)
    emb = np.zeros(arrs["b_time_out"].shape[0], np.float32)
    rc = load().orc_dit_input_forward(ctypes.byref(cfg), _p(video), _p(text), text.shape[0], ctypes.c_float(timestep),
                                      T, H, W, _p(vo), _p(to), _p(emb))
    if rc != 0:
        raise RuntimeError(f"orc_dit_input_forward failed: {rc}")
    return vo, to, emb


def dit_output_forward(weights, vid, emb, T, h, w, *, eps=1e-5, threads=0):
    """The DiT output head.  weights: {field: array} of OUTPUT_FIELDS; vid
    [T*h*w, dim].  Returns [T*2h*2w, output_channels] token-major."""
    arrs = {k: _f32(weights[k]) for k in OUTPUT_FIELDS}
    vid, emb = _f32(vid), _f32(emb)
    dim = vid.shape[1]
    oc = arrs["b_proj"].shape[0] // 4
    cfg = OrcDitOutput(dim, oc, eps, *[_p(arrs[k]) for k in OUTPUT_FIELDS], threads)
    out = np.zeros((T * 4 * h * w, oc), np.float32)
    rc = load().orc_dit_output_forward(ctypes.byref(cfg), _p(vid), _p(emb), T, h, w, _p(out))
    if rc != 0:
        raise RuntimeError(f"orc_dit_output_forward failed: {rc}")
    return out


def dit_forward(input_weights, blocks, output_weights, latent, text, timestep, *, eps=1e-5, threads=0):
    """SeedVR2DiT::forward (dit.cpp:281-383) composed from the oracle's heads
    and blocks.  latent [C, T, H, W] fp32 (channel-major, as the engine holds
    it), blocks: Block objects in order.  Returns [16, T, H, W]."""
    C, T, H, W = latent.shape
    flat = np.ascontiguousarray(np.transpose(latent, (1, 2, 3, 0)).reshape(T * H * W, C))  # dit.cpp:66-80
    vid, txt, emb = dit_input_forward(input_weights, flat, text, timestep, T, H, W, threads=threads)
    for blk in blocks:
        vid, txt = blk.forward(vid, txt, emb, T, H // 2, W // 2)
    out = dit_output_forward(output_weights, vid, emb, T, H // 2, W // 2, eps=eps, threads=threads)
    oc = out.shape[1]
    return np.ascontiguousarray(np.transpose(out.reshape(T, H, W, oc), (3, 0, 1, 2)))  # dit.cpp:82-95


# ---- Euler sampler (src/model/sampler.cpp, src/core/engine.cpp) -----------

def euler_timesteps(steps):
    """EulerSampler(steps).timesteps() (sampler.cpp:181-187)."""
    out = np.zeros(max(1, steps), np.float32)
    n = load().orc_euler_timesteps(steps, _p(out))
    return out[:n]


def condition_ratio(noise_scale, T, H, W):
    """transformed_condition_timestep / 1000 (engine.cpp:79-92, :110)."""
    return load().orc_condition_ratio(noise_scale, T, H, W)


def make_condition(encoded, noise, ratio):
    """make_condition_latent (engine.cpp:106-122), any shape."""
    a, b = _f32(encoded), _f32(noise)
    out = np.empty_like(a)
    load().orc_make_condition(_p(a), _p(b), _p(out), a.size, ratio)
    return out


def make_dit_input(latent, condition, channel_major=True):
    """make_dit_input (engine.cpp:125-149): [16, T, H, W] -> [33, T, H, W];
    channel_major=False: [tokens, 16] -> [tokens, 33] (sampler.cpp:337-357)."""
    a, b = _f32(latent), _f32(condition)
    if channel_major:
        tokens = a.size // 16
        out = np.empty((33,) + a.shape[1:], np.float32)
    else:
        tokens = a.shape[0]
        out = np.empty((tokens, 33), np.float32)
    load().orc_make_dit_input(_p(a), _p(b), _p(out), tokens, 1 if channel_major else 0)
    return out


def standard_deviation(x):
    """standard_deviation (sampler.cpp:41-62)."""
    a = _f32(x)
    return load().orc_standard_deviation(_p(a), a.size)


def apply_cfg(positive, negative, scale, rescale):
    """EulerSampler::apply_cfg (sampler.cpp:201-236)."""
    a, b = _f32(positive), _f32(negative)
    out = np.empty_like(a)
    load().orc_apply_cfg(_p(a), _p(b), _p(out), a.size, scale, rescale)
    return out


def euler_step(prediction, current, timestep, next_timestep):
    """EulerSampler::step_to (sampler.cpp:239-265)."""
    a, b = _f32(prediction), _f32(current)
    out = np.empty_like(b)
    load().orc_euler_step(_p(a), _p(b), _p(out), b.size, timestep, next_timestep)
    return out


def euler_endpoint(prediction, current, timestep):
    """EulerSampler::endpoint (sampler.cpp:267-285)."""
    a, b = _f32(prediction), _f32(current)
    out = np.empty_like(b)
    load().orc_euler_endpoint(_p(a), _p(b), _p(out), b.size, timestep)
    return out
