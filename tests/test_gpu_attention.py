"""GPU parity of the windowed joint attention (sv2_window_attention) against
the CPU oracle on identical seeded inputs.

Cases: the single-layer shapes of the benchmark configurations (grid 2x16x30,
20 heads, 58 text tokens, 2x8x10 windows, unshifted and shifted), the
reference's adaptive windows (no explicit size), the 720p grid 6x45x80 with
2x9x16 windows (every video and text output of both plans), the four small cases of the reference's own CPU-vs-Vulkan block
test (tests/dit_block_vulkan_runner.cpp:213-218) at the attention level, and
edge cases (one token, no text tokens).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch  # noqa: F401  (first import is slow on a fresh box; keep it out of test timeouts)

from attn_case import run_attention_case as _case
from parity import reference_freqs

pytestmark = pytest.mark.gpu

L_TXT = 58  # embeddings/default_pos_emb.bin header [58, 5120]


def test_single_layer_2x16x30_unshifted_no_norm_no_rope(hip, orc, device):
    # the CPU-reference layer shape: windows 2x8x10 (6), no RoPE, no QK-norm
    _case(hip, orc, device, T=2, H=16, W=30, Lt=L_TXT, heads=20, wt=2, wh=8, ww=10,
          qk_norm=False, rope_mode=2, in_dtype="f32", out_dtype="f32", seed=1)


@pytest.mark.parametrize("shifted", [False, True], ids=["unshifted", "shifted"])
def test_single_layer_2x16x30_fp32_norm_rope_flip_rate(hip, orc, device, shifted):
    # the fp32 parity mode at the config-2 shape: P enters P*V as three bf16
    # terms against exact bf16 V, so the pre-rounding values are fp32-class
    # and a bf16 rounding flip against the oracle is rare (< 0.1%; fp16 P flips
    # about 8% of the elements)
    rep_v, _ = _case(hip, orc, device, T=2, H=16, W=30, Lt=L_TXT, heads=20, shifted=shifted, wt=2, wh=8, ww=10,
                     qk_norm=True, rope_mode=0, in_dtype="f32", out_dtype="f32", seed=6 + shifted)
    assert rep_v["flips"] <= 1e-3 * rep_v["n"], rep_v
    assert rep_v["pre_max_abs"] <= 1e-5, rep_v


def test_single_layer_2x16x30_fp16_shifted_norm_rope(hip, orc, device):
    # fp16 layer with QK-norm and RoPE, shifted (0,4,5) ragged windows (12)
    _case(hip, orc, device, T=2, H=16, W=30, Lt=L_TXT, heads=20, shifted=True, wt=2, wh=8, ww=10,
          qk_norm=True, rope_mode=0, in_dtype="f16", out_dtype="f16", seed=2)


def test_single_layer_2x16x30_absolute_rope(hip, orc, device):
    _case(hip, orc, device, T=2, H=16, W=30, Lt=L_TXT, heads=20, shifted=True, wt=2, wh=8, ww=10,
          qk_norm=True, rope_mode=1, in_dtype="f16", out_dtype="bf16", seed=3)


@pytest.mark.parametrize("shifted", [False, True])
def test_reference_adaptive_windows(hip, orc, device, shifted):
    # no explicit window size: the reference's adaptive rule (1x15x28 here)
    _case(hip, orc, device, T=2, H=16, W=30, Lt=L_TXT, heads=4, shifted=shifted,
          in_dtype="bf16", out_dtype="f32", seed=4 + shifted)


@pytest.mark.parametrize("shifted", [False, True])
def test_720p_grid_all_windows(hip, orc, device, shifted):
    # 6x45x80 with 2x9x16 windows (75 / 144, the shifted plan's ragged
    # interior and edge windows included): every video and text output
    # against the oracle
    _case(hip, orc, device, T=6, H=45, W=80, Lt=L_TXT, heads=20, shifted=shifted, wt=2, wh=9, ww=16,
          in_dtype="f16", out_dtype="f16", seed=10 + shifted)


@pytest.mark.parametrize("case", [
    # tests/dit_block_vulkan_runner.cpp:213-218 at the attention level
    dict(T=2, H=2, W=2, Lt=3, heads=1, shifted=False),
    dict(T=2, H=2, W=2, Lt=3, heads=1, shifted=True),
    dict(T=1, H=1, W=1, Lt=2, heads=1, shifted=False),
    dict(T=3, H=2, W=2, Lt=4, heads=2, shifted=False),
])
def test_reference_runner_shapes(hip, orc, device, case):
    _case(hip, orc, device, **case, in_dtype="f32", out_dtype="f32", seed=20)


def test_no_text_tokens(hip, orc, device):
    _case(hip, orc, device, T=2, H=5, W=7, Lt=0, heads=2, shifted=True, wt=1, wh=2, ww=3,
          in_dtype="f16", out_dtype="f32", seed=30)


def test_long_text_many_key_blocks(hip, orc, device):
    # S spans several 64-key blocks and 128-query blocks with ragged tails
    _case(hip, orc, device, T=3, H=7, W=9, Lt=150, heads=3, shifted=True, wt=2, wh=4, ww=5,
          in_dtype="f16", out_dtype="f32", seed=31)


def test_index_map_bitexact(hip, orc, device):
    import torch
    for (T, H, W, sh, wt, wh, ww) in [(2, 16, 30, False, 2, 8, 10), (2, 16, 30, True, 2, 8, 10),
                                      (6, 45, 80, True, 2, 9, 16), (6, 45, 80, False, 0, 0, 0),
                                      (2, 16, 30, True, 0, 0, 0), (5, 7, 3, True, 2, 2, 2)]:
        print(f"[index map] {T}x{H}x{W} shifted={sh} win=({wt},{wh},{ww})", flush=True)
        out = torch.full((T * H * W,), -1, dtype=torch.int32, device=device)
        hip.window_index_map(hip.rule(T, H, W, sh, wt, wh, ww), out)
        torch.cuda.synchronize()
        ref = [((t * H + y) * W + x) for (t0, t1, h0, h1, w0, w1) in orc.make_windows(T, H, W, sh, wt, wh, ww)
               for t in range(t0, t1) for y in range(h0, h1) for x in range(w0, w1)]
        assert np.array_equal(out.cpu().numpy(), np.array(ref, dtype=np.int32))


@pytest.mark.parametrize("rope_mode,in_dtype", [(0, "f16"), (0, "f32"), (1, "f32"), (2, "bf16"), (0, "bf16")])
def test_prologue_matches_oracle(hip, orc, device, rope_mode, in_dtype):
    """q/k/v after norm, rotation and bf16 rounding, through the same device
    code the attention kernel runs.  The RoPE table holds the host C library's
    cosf/sinf, exactly the reference's values.
    fp32 and bf16 inputs (the exact prologue): double sum of squares, float of
    its mean, correctly rounded fp32 sqrt and divide, unfused products, as the
    reference evaluates them; q and k are bit-identical to the oracle's (the
    double sums run in another order, which changes the float mean only when
    the sum lies within ~2^-50 of a rounding boundary: a handful of elements
    at most is allowed).
    fp16 inputs (the fast prologue): fp32 sum of squares, the hardware
    reciprocal square root and one product fused into each RoPE add; an
    element may then round to the neighbouring bf16 value (one ulp) — rare —
    and where the rotation cancels (a*c - b*s near 0) the tiny result can move
    by a few of its own ulps, bounded here by 1e-6 absolute on O(1) data.
    v is compared as
    the operand the kernel feeds the P*V MFMA.  fp32 and bf16 inputs: the bf16
    value itself, bit for bit.  fp16 inputs: fp16 of the bf16 value, exact
    except in fp16's subnormal range (|v| < 2^-14), where the kernel's
    conversion rounds toward zero (at most one fp16 subnormal step, 2^-24)."""
    import torch
    T, H, W, Lt, heads = 2, 16, 30, L_TXT, 4
    print(f"[prologue] rope={rope_mode} in={in_dtype}", flush=True)
    rng = np.random.default_rng(40 + rope_mode)
    D = heads * 128
    vid = rng.standard_normal((T * H * W, 3 * D), dtype=np.float32) * 3
    txt = rng.standard_normal((Lt, 3 * D), dtype=np.float32) * 3
    tdt = {"f16": torch.float16, "f32": torch.float32, "bf16": torch.bfloat16}[in_dtype]
    vid = torch.from_numpy(vid).to(tdt).float().numpy()
    txt = torch.from_numpy(txt).to(tdt).float().numpy()
    gam = rng.uniform(0.5, 1.5, (4, 128)).astype(np.float32)
    freqs = reference_freqs()
    _, _, caps = orc.window_attention(vid, txt, T, H, W, heads=heads, rope_mode=rope_mode, freqs=freqs,
                                      gammas=list(gam), shifted=True, wt=2, wh=8, ww=10, capture=True)
    attn = hip.WindowAttention(hip.rule(T, H, W, True, 2, 8, 10), heads, Lt, rope_mode=rope_mode,
                               freqs=freqs, device=device)
    outs = [torch.full(caps["q"].shape, float("nan"), device=device) for _ in range(3)]
    attn.prologue(torch.from_numpy(vid).to(device, tdt), torch.from_numpy(txt).to(device, tdt),
                  [torch.from_numpy(g).to(device) for g in gam], *outs)
    torch.cuda.synchronize()
    v_expect = caps["v"].astype(np.float16).astype(np.float32) if in_dtype == "f16" else caps["v"]
    expect = {"q": caps["q"], "k": caps["k"], "v": v_expect}
    for name, o in zip("qkv", outs):
        g = o.cpu().numpy()
        r = expect[name]
        assert np.isfinite(g).all()
        differ = g.view(np.uint32) != r.view(np.uint32)
        frac = differ.mean()
        print(f"  {name}: {int(differ.sum())} of {g.size} differ", flush=True)
        if name == "v":
            if in_dtype != "f16":
                assert not differ.any()
                continue
            tiny = np.abs(r) < 2.0 ** -14
            assert not (differ & ~tiny).any()
            assert (np.abs(g[differ].astype(np.float64) - r[differ]) <= 2.0 ** -24).all()
            continue
        if in_dtype != "f16":
            assert int(differ.sum()) <= 4, f"{name}: {int(differ.sum())} elements differ in the exact prologue"
        assert frac <= 2e-3, f"{name}: {frac:.2e} of the elements differ"
        if differ.any():
            d = np.abs(g[differ].astype(np.float64) - r[differ])
            ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(g[differ]), np.abs(r[differ])))[1] - 8)
            assert ((d <= ulp * 1.000001) | (d <= 1e-6)).all()


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_stages_one_at_a_time_equal_the_combined_call(hip, device, dtype):
    """sv2_window_attention_stages: the text prologue, the window kernel and
    the text reduction launched one call each (and the first two together)
    give the combined call's outputs bit for bit."""
    import torch
    print(f"[stages] {dtype}", flush=True)
    T, H, W, heads = 2, 16, 30, 20
    D = heads * 128
    tdt = torch.float16 if dtype == "f16" else torch.float32
    g = torch.Generator(device=device)
    g.manual_seed(77)
    vid = torch.randn((T * H * W, 3 * D), generator=g, device=device).to(tdt)
    txt = torch.randn((L_TXT, 3 * D), generator=g, device=device).to(tdt)
    gam = [torch.rand(128, generator=g, device=device) + 0.5 for _ in range(4)]
    attn = hip.WindowAttention(hip.rule(T, H, W, True, 2, 8, 10), heads, L_TXT, freqs=reference_freqs(),
                               device=device)

    def outs():
        return (torch.full((T * H * W, D), float("nan"), dtype=tdt, device=device),
                torch.full((L_TXT, D), float("nan"), dtype=tdt, device=device))

    ref_v, ref_t = outs()
    attn(vid, txt, gam, ref_v, ref_t)
    for split in ([hip.STAGE_TEXT_PREPARE, hip.STAGE_WINDOWS, hip.STAGE_TEXT_REDUCE],
                  [hip.STAGE_TEXT_PREPARE | hip.STAGE_WINDOWS, hip.STAGE_TEXT_REDUCE]):
        ov, ot = outs()
        attn.workspace.fill_(255)  # the stages must rebuild what the combined call left there
        for st in split:
            attn(vid, txt, gam, ov, ot, stages=st)
        torch.cuda.synchronize()
        assert torch.equal(ov, ref_v), split
        assert torch.equal(ot, ref_t), split
