"""The C ABI without a GPU: the library loads, exports every function
include/seedvr2_hip.h declares, and its host-only entry points (window plan,
RoPE table, argument checks) behave as the reference's layer does.  No
device work is launched here."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import winplan_exact as wx
from parity import reference_freqs

REPO = Path(__file__).resolve().parent.parent


def declared_functions() -> list[str]:
    names = []
    for hdr in sorted((REPO / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", hdr.read_text(), flags=re.S)
        names += re.findall(r"\b(sv2_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_function(hip):
    lib = hip.load()
    decl = declared_functions()
    assert len(decl) >= 12
    missing = [n for n in decl if not hasattr(lib, n)]
    assert not missing, missing
    assert set(decl) == set(hip.EXPORTS) | (set(decl) - set(hip.EXPORTS))
    assert not set(hip.EXPORTS) - set(decl), "binding lists a function the header does not declare"


def test_version_and_error_string(hip):
    lib = hip.load()
    assert b"gfx950" in lib.sv2_version()
    assert isinstance(lib.sv2_last_error(), bytes)


@pytest.mark.parametrize("args", [
    (2, 16, 30, False, 2, 8, 10), (2, 16, 30, True, 2, 8, 10), (6, 45, 80, False, 2, 9, 16),
    (6, 45, 80, True, 2, 9, 16), (2, 16, 30, True, 0, 0, 0), (6, 45, 80, True, 0, 0, 0),
    (5, 7, 3, True, 2, 2, 2), (1, 1, 1, True, 0, 0, 0), (21, 90, 160, True, 0, 0, 0),
])
def test_window_plan_matches_reference_rule(hip, args):
    assert hip.window_plan(hip.rule(*args)) == wx.plan(*args)


def test_window_plan_brute_force(hip):
    for T in range(1, 6):
        for H in range(1, 11):
            for W in range(1, 11):
                for sh in (False, True):
                    for win in ((0, 0, 0), (2, 3, 4), (1, 4, 3)):
                        assert hip.window_plan(hip.rule(T, H, W, sh, *win)) == wx.plan(T, H, W, sh, *win)


def test_window_plan_rejects_bad_rules(hip):
    lib = hip.load()
    for bad in [hip.rule(0, 4, 4), hip.rule(2, -1, 4), hip.rule(2, 4, 4, False, -1, 0, 0)]:
        assert lib.sv2_window_plan(ctypes.byref(bad), None, 0) == hip.SV2_EINVAL
    assert lib.sv2_window_plan(None, None, 0) == hip.SV2_EINVAL
    # the first `cap` windows only
    r = hip.rule(2, 16, 30, True, 2, 8, 10)
    arr = (hip.Window * 3)()
    assert lib.sv2_window_plan(ctypes.byref(r), arr, 3) == 12
    assert [(w.t0, w.t1, w.h0, w.h1, w.w0, w.w1) for w in arr] == wx.plan(2, 16, 30, True, 2, 8, 10)[:3]


def test_rope_table_reference_mode(hip):
    freqs = reference_freqs()
    npos = 70
    tab = hip.rope_table(hip.ROPE_REFERENCE, freqs, 10000.0, npos).reshape(3, npos, 24, 2)
    pos = np.arange(npos, dtype=np.float32)[:, None]
    ang = (pos * freqs[None, :]).astype(np.float32)  # float(pos) * freq in fp32, as the reference forms it
    for a in range(3):
        assert np.allclose(tab[a, :, :21, 0], np.cos(ang.astype(np.float64)), atol=2e-7)
        assert np.allclose(tab[a, :, :21, 1], np.sin(ang.astype(np.float64)), atol=2e-7)
        # slots past the 21 pairs rotate by zero
        assert (tab[a, :, 21:, 0] == 1).all() and (tab[a, :, 21:, 1] == 0).all()


def test_rope_table_absolute_mode(hip):
    npos = 40
    tab = hip.rope_table(hip.ROPE_ABSOLUTE, None, 10000.0, npos).reshape(3, npos, 24, 2)
    for a, n in enumerate((32, 48, 48)):
        fr = (1.0 / 10000.0 ** (np.arange(0, n, 2) / n)).astype(np.float32)
        ang = (np.arange(npos, dtype=np.float32)[:, None] * fr[None, :]).astype(np.float64)
        assert np.allclose(tab[a, :, :n // 2, 0], np.cos(ang), atol=2e-7)
        assert np.allclose(tab[a, :, :n // 2, 1], np.sin(ang), atol=2e-7)


def test_rope_positions_needed(hip):
    # reference mode: video t positions reach L_txt + window_t - 1
    assert hip.rope_positions_needed(hip.rule(6, 45, 80, True, 2, 9, 16), 58, hip.ROPE_REFERENCE) == 60
    assert hip.rope_positions_needed(hip.rule(2, 16, 30, False, 2, 8, 10), 0, hip.ROPE_REFERENCE) == 10
    assert hip.rope_positions_needed(hip.rule(6, 45, 80, True, 2, 9, 16), 58, hip.ROPE_ABSOLUTE) == 80


def test_attention_argument_checks(hip):
    """Invalid arguments are rejected on the host before any launch (the
    reference layer returns -1 for bad blobs, seedvr2_dit_block.cpp:1119-1138)."""
    lib = hip.load()
    a = hip.AttnArgs()
    a.rule = hip.rule(2, 16, 30, False, 2, 8, 10)
    a.heads, a.head_dim, a.text_len, a.eps = 20, 128, 58, 1e-5
    a.rope_mode = hip.ROPE_NONE
    a.qk_norm = 0
    a.vid_qkv = 16
    a.txt_qkv = 16
    a.qkv_dtype = hip.F16
    a.out_dtype = hip.F16
    assert lib.sv2_window_attention_workspace(ctypes.byref(a)) > 0
    a.head_dim = 64
    assert lib.sv2_window_attention_workspace(ctypes.byref(a)) == hip.SV2_EUNSUPPORTED
    a.head_dim = 128
    a.qkv_dtype = 7
    assert lib.sv2_window_attention_workspace(ctypes.byref(a)) == hip.SV2_EINVAL
    a.qkv_dtype = hip.F16
    a.rope_mode = hip.ROPE_REFERENCE  # no table
    assert lib.sv2_window_attention(ctypes.byref(a), None) == hip.SV2_EINVAL
    assert b"rope" in lib.sv2_last_error()
    a.rope_mode = hip.ROPE_NONE
    a.qk_norm = 1  # no gammas
    assert lib.sv2_window_attention(ctypes.byref(a), None) == hip.SV2_EINVAL
    a.qk_norm = 0
    # outputs missing
    assert lib.sv2_window_attention(ctypes.byref(a), None) == hip.SV2_EINVAL
    assert lib.sv2_window_attention(None, None) == hip.SV2_EINVAL


def test_attention_stage_checks(hip):
    """sv2_window_attention_stages takes a non-empty set of the three stage
    bits, checks the arguments as sv2_window_attention does, and runs the
    exact mode's stages only together; all rejected on the host."""
    lib = hip.load()
    a = hip.AttnArgs()
    a.rule = hip.rule(2, 16, 30, False, 2, 8, 10)
    a.heads, a.head_dim, a.text_len, a.eps = 20, 128, 58, 1e-5
    a.rope_mode = hip.ROPE_NONE
    a.qk_norm = 0
    a.vid_qkv = a.txt_qkv = 16
    a.qkv_dtype = a.out_dtype = hip.F16
    for bad in (0, 8, 9, -1):
        assert lib.sv2_window_attention_stages(ctypes.byref(a), bad, None) == hip.SV2_EINVAL, bad
        assert b"stages" in lib.sv2_last_error()
    # outputs missing: the same check as the combined call
    assert lib.sv2_window_attention_stages(ctypes.byref(a), hip.STAGE_WINDOWS, None) == hip.SV2_EINVAL
    assert b"output" in lib.sv2_last_error()
    a.vid_out = a.txt_out = 16
    a.qkv_dtype = a.out_dtype = hip.F32
    a.exact = 1
    for partial in (hip.STAGE_TEXT_PREPARE, hip.STAGE_WINDOWS, hip.STAGE_TEXT_REDUCE, 3, 6):
        assert lib.sv2_window_attention_stages(ctypes.byref(a), partial, None) == hip.SV2_EUNSUPPORTED, partial
    assert (hip.STAGE_TEXT_PREPARE | hip.STAGE_WINDOWS | hip.STAGE_TEXT_REDUCE) == hip.STAGE_ALL


def test_workspace_size_formula(hip):
    """Per-window bf16 text partials, the prepared text q, k and v^T, and the
    first two text tiles' v^T per head in the attention kernel's LDS byte
    order."""
    lib = hip.load()
    a = hip.AttnArgs()
    a.rule = hip.rule(6, 45, 80, True, 2, 9, 16)
    a.heads, a.head_dim, a.text_len, a.eps = 20, 128, 58, 1e-5
    a.rope_mode = hip.ROPE_NONE
    a.vid_qkv = a.txt_qkv = 16
    a.qkv_dtype = a.out_dtype = hip.F16
    got = lib.sv2_window_attention_workspace(ctypes.byref(a))
    D = 20 * 128

    def al(x):
        return (x + 255) // 256 * 256
    expect = al(144 * 58 * D * 2) + al(20 * 58 * 128 * 2) * 2 + al(20 * 128 * 64 * 2) + al(20 * 2 * 64 * 128 * 2)
    assert got == expect
    a.text_len = 0
    assert lib.sv2_window_attention_workspace(ctypes.byref(a)) == 0


def test_elementwise_argument_checks(hip):
    """Shape and pointer checks of the elementwise entry points return before
    any launch."""
    lib = hip.load()
    f = ctypes.c_float(1e-5)
    assert lib.sv2_rmsnorm_ada(16, 16, hip.F16, 4, 12, f, None, None, None, 0, 0, None) == hip.SV2_EUNSUPPORTED
    assert lib.sv2_rmsnorm_ada(16, 16, hip.F16, 4, 8192, f, None, None, None, 0, 0, None) == hip.SV2_EUNSUPPORTED
    assert lib.sv2_rmsnorm_ada(16, 16, 9, 4, 2560, f, None, None, None, 0, 0, None) == hip.SV2_EINVAL
    assert lib.sv2_rmsnorm_ada(16, 16, hip.F16, 4, 2560, f, None, None, None, 0, 1, None) == hip.SV2_EINVAL
    assert lib.sv2_rmsnorm_ada(16, 16, hip.F16, 4, 2560, f, 16, 16, 16, 1, 1, None) == hip.SV2_EINVAL
    assert lib.sv2_rmsnorm_ada(None, None, hip.F16, 0, 2560, f, None, None, None, 0, 0, None) == hip.SV2_OK
    assert lib.sv2_ada_residual(16, 16, hip.F16, 4, 2560, None, None, 0, 3, None) == hip.SV2_EINVAL
    assert lib.sv2_ada_residual(16, None, hip.F16, 4, 2560, None, None, 0, 1, None) == hip.SV2_EINVAL
    assert lib.sv2_ada_residual(16, 16, hip.F16, 4, 2560, None, None, 0, 0, None) == hip.SV2_EINVAL
    assert lib.sv2_swiglu(16, 16, hip.F16, 12, None) == hip.SV2_EUNSUPPORTED
    assert lib.sv2_swiglu(None, 16, hip.F16, 16, None) == hip.SV2_EINVAL
    assert lib.sv2_swiglu(None, None, hip.F16, 0, None) == hip.SV2_OK


def test_inner_product_argument_checks(hip):
    """Shape, pointer and size checks of the InnerProduct entry points return
    before any launch: the hand-written fp16 product needs in % 64 == 0 and
    out % 256 == 0 (SwiGLU: % 128), and refuses operands past 2 GiB (its
    buffer resources take 32-bit byte offsets); the fp32 exact product needs
    positive sizes."""
    lib = hip.load()
    p = 16  # a non-null dummy address: every case below returns before touching it
    f16 = lib.sv2_inner_product_f16
    assert f16(p, p, None, p, 4, 48, 256, hip.EPI_STORE, None, None, None, None) == hip.SV2_EUNSUPPORTED
    assert f16(p, p, None, p, 4, 64, 200, hip.EPI_STORE, None, None, None, None) == hip.SV2_EUNSUPPORTED
    assert f16(p, p, p, p, 4, 64, 192, hip.EPI_SWIGLU, None, None, None, None) == hip.SV2_EUNSUPPORTED
    assert f16(p, p, None, p, 4, 64, 256, 7, None, None, None, None) == hip.SV2_EINVAL
    assert f16(None, p, None, p, 4, 64, 256, hip.EPI_STORE, None, None, None, None) == hip.SV2_EINVAL
    assert f16(p, p, None, p, 4, 64, 256, hip.EPI_RESIDUAL, None, None, None, None) == hip.SV2_EINVAL
    assert f16(p, p, None, p, 4, 64, 256, hip.EPI_SWIGLU, None, None, None, None) == hip.SV2_EINVAL
    assert f16(p, p, p, p, 4, 64, 256, hip.EPI_STORE, None, None, None, None) == hip.SV2_EINVAL
    # 2^24 rows x 64 in x 2 B = 2 GiB of X; 65536 outputs x 16384 in x 2 B = 2 GiB of W
    assert f16(p, p, None, p, 1 << 24, 64, 256, hip.EPI_STORE, None, None, None, None) == hip.SV2_EUNSUPPORTED
    assert "2 GiB" in lib.sv2_last_error().decode()
    assert f16(p, p, None, p, 4, 16384, 65536, hip.EPI_STORE, None, None, None, None) == hip.SV2_EUNSUPPORTED
    assert f16(None, None, None, None, 0, 64, 256, hip.EPI_STORE, None, None, None, None) == hip.SV2_OK
    f32 = lib.sv2_inner_product_f32
    assert f32(p, p, None, p, 4, 0, 16, None) == hip.SV2_EINVAL
    assert f32(p, p, None, p, -1, 16, 16, None) == hip.SV2_EINVAL
    assert f32(None, p, None, p, 4, 16, 16, None) == hip.SV2_EINVAL
    assert f32(None, None, None, None, 0, 16, 16, None) == hip.SV2_OK


def test_few_row_inner_product_checks(hip):
    """The few-row fp16 InnerProduct (sv2_inner_product_f16_few) checks its
    shape, epilogue, pointers and workspace before any launch, and sizes its
    split partial sums: 6 splits of 58 x 2560 fp32 for the 2560 -> 2560 and
    6912 -> 2560 products (40 column tiles), 2 of 58 x 7680 for 2560 -> 7680
    (120 tiles), none for SwiGLU."""
    lib = hip.load()
    ws = lib.sv2_inner_product_f16_few_workspace
    assert ws(58, 2560, 2560, hip.EPI_RESIDUAL) == 6 * 58 * 2560 * 4
    assert ws(58, 6912, 2560, hip.EPI_RESIDUAL) == 6 * 58 * 2560 * 4
    assert ws(58, 2560, 7680, hip.EPI_STORE) == 2 * 58 * 7680 * 4
    assert ws(58, 2560, 6912, hip.EPI_SWIGLU) == 0
    assert ws(1, 64, 64, hip.EPI_STORE) == 0          # one K block: never split
    assert ws(0, 2560, 2560, hip.EPI_STORE) == 0
    assert ws(65, 2560, 2560, hip.EPI_STORE) == hip.SV2_EUNSUPPORTED
    assert ws(58, 2560, 2560, 9) == hip.SV2_EINVAL
    p = 16  # a non-null dummy address: every case below returns before touching it
    f = lib.sv2_inner_product_f16_few
    args = (None, None, None, None)
    assert f(p, p, None, p, 65, 64, 64, hip.EPI_STORE, *args, 0, None) == hip.SV2_EUNSUPPORTED
    assert f(p, p, None, p, 8, 48, 64, hip.EPI_STORE, *args, 0, None) == hip.SV2_EUNSUPPORTED
    assert f(p, p, None, p, 8, 64, 96, hip.EPI_STORE, *args, 0, None) == hip.SV2_EUNSUPPORTED
    assert f(p, p, p, p, 8, 64, 48, hip.EPI_SWIGLU, *args, 0, None) == hip.SV2_EUNSUPPORTED
    assert f(p, p, None, p, 8, 64, 64, 5, *args, 0, None) == hip.SV2_EINVAL
    assert f(None, p, None, p, 8, 64, 64, hip.EPI_STORE, *args, 0, None) == hip.SV2_EINVAL
    assert f(p, p, None, p, 8, 64, 64, hip.EPI_RESIDUAL, *args, 0, None) == hip.SV2_EINVAL
    assert f(p, p, None, p, 8, 64, 64, hip.EPI_SWIGLU, *args, 0, None) == hip.SV2_EINVAL
    assert f(p, p, p, p, 8, 64, 64, hip.EPI_STORE, *args, 0, None) == hip.SV2_EINVAL
    assert f(p, p, p, p, 8, 64, 64, hip.EPI_SWIGLU, p, None, None, None, 0, None) == hip.SV2_EINVAL
    # a split product without (or with too small) a workspace
    assert f(p, p, None, p, 58, 2560, 2560, hip.EPI_STORE, None, None, None, None, 0, None) == hip.SV2_EINVAL
    assert f(p, p, None, p, 58, 2560, 2560, hip.EPI_STORE, None, None, None, p, 1000, None) == hip.SV2_EINVAL
    assert "workspace" in lib.sv2_last_error().decode()
    assert f(None, None, None, None, 0, 64, 64, hip.EPI_STORE, *args, 0, None) == hip.SV2_OK


def test_misaligned_device_pointers_are_refused(hip):
    """Operands the kernels fetch straight into LDS (or with 16-byte vector
    loads) must be aligned: a misaligned qkv, output or workspace pointer of
    the attention, or operand of the InnerProducts, is refused before any
    launch (these dummy addresses are never touched)."""
    lib = hip.load()
    a16, a8, odd = 4096, 4104, 4098
    f = lib.sv2_inner_product_f16
    assert f(odd, a16, None, a16, 4, 64, 256, hip.EPI_STORE, None, None, None, None) == hip.SV2_EINVAL
    assert f(a16, a8, None, a16, 4, 64, 256, hip.EPI_STORE, None, None, None, None) == hip.SV2_EINVAL
    assert f(a16, a16, None, a8, 4, 64, 256, hip.EPI_STORE, None, None, None, None) == hip.SV2_EINVAL
    assert "aligned" in lib.sv2_last_error().decode()
    g = lib.sv2_inner_product_f16_few
    assert g(a8, a16, None, a16, 4, 64, 64, hip.EPI_STORE, None, None, None, None, 0, None) == hip.SV2_EINVAL
    assert g(a16, a16, None, odd, 4, 64, 64, hip.EPI_STORE, None, None, None, None, 0, None) == hip.SV2_EINVAL
    assert g(a16, a16, None, a16, 4, 64, 64, hip.EPI_RESIDUAL, None, None, odd, None, 0, None) == hip.SV2_EINVAL
    assert "aligned" in lib.sv2_last_error().decode()
    # attention: the size query takes any 16-byte-aligned placeholder, and
    # refuses a misaligned qkv pointer
    args = hip.AttnArgs()
    args.rule = hip.rule(2, 16, 30, False, 2, 8, 10)
    args.heads, args.head_dim, args.text_len = 2, 128, 8
    args.eps, args.qk_norm, args.rope_mode = 1e-5, 0, hip.ROPE_NONE
    args.qkv_dtype = args.out_dtype = hip.F16
    args.vid_qkv = args.txt_qkv = a16
    assert lib.sv2_window_attention_workspace(ctypes.byref(args)) >= 0
    args.txt_qkv = a8
    assert lib.sv2_window_attention_workspace(ctypes.byref(args)) == hip.SV2_EINVAL
    assert "aligned" in lib.sv2_last_error().decode()
