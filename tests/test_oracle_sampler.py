"""Pins the oracle's Euler sampler and latent preparation (oracle/refcpu.c,
orc_euler_* / orc_apply_cfg / orc_make_*) on the CPU, and the host half of
the library's sampler ABI:
  * the reference's own known answers: CFG 1.5 of (2, 0) is 3 and the
    endpoint of x = 1, pred = 0.25 at t = 1000 is 0.75 (tests/
    runtime_unit_test.cpp:61-77); the condition ratio 0.25 mix, the
    token-major 33-channel layout, CFG 2.5 / rescale 0.4 and the 1000 -> 500
    step on the 7-token pattern of tests/sampler_vulkan_runner.cpp:66-148;
  * float64 closed forms: CFG with the rescale against numpy std(ddof=1),
    the v-lerp step against its expanded form x + (bs - bt) * pred, the
    timestep schedule 1000 * (1 - i / n), the condition-ratio shift at the
    two resolutions where it reduces to t and 5t / (1 + 4t);
  * identities that a dropped term or swapped operand breaks: scale 0 gives
    the negative, rescale 1 gives std(out) = std(pos), the endpoint equals the
    step to t_next = 0 bit for bit, t_next beyond 1000 clamps to 1000, a
    constant CFG output skips the rescale.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest


def _pattern(tokens=7):
    i = np.arange(16 * tokens)
    pos = ((i % 13 - 6).astype(np.float32) * np.float32(0.07)).astype(np.float32)
    neg = ((i % 9 - 4).astype(np.float32) * np.float32(0.05)).astype(np.float32)
    return pos.reshape(tokens, 16), neg.reshape(tokens, 16)


def test_reference_unit_known_answers(orc):
    cfg = orc.apply_cfg(np.full(2, 2.0), np.zeros(2), 1.5, 0.0)
    assert np.all(cfg == 3.0)
    end = orc.euler_endpoint(np.full(2, 0.25), np.ones(2), 1000.0)
    assert np.all(end == 0.75)


def test_reference_runner_condition_and_layout(orc):
    pos, neg = _pattern()
    cond = orc.make_condition(pos, neg, 0.25)
    expected = 0.75 * pos.astype(np.float64) + 0.25 * neg.astype(np.float64)
    assert np.max(np.abs(cond - expected)) <= 1e-6
    dit = orc.make_dit_input(pos, cond, channel_major=False)
    assert dit.shape == (7, 33)
    assert np.array_equal(dit[:, :16], pos)
    assert np.array_equal(dit[:, 16:32], cond)
    assert np.all(dit[:, 32] == 1.0)


def test_reference_runner_cfg_and_step(orc):
    pos, neg = _pattern()
    cfg = orc.apply_cfg(pos, neg, 2.5, 0.4)
    p64, n64 = pos.astype(np.float64), neg.astype(np.float64)
    raw = n64 + 2.5 * (p64 - n64)
    factor = 0.4 * np.std(p64, ddof=1) / np.std(raw, ddof=1) + 0.6
    assert np.max(np.abs(cfg - raw * factor)) <= 2e-5
    nxt = orc.euler_step(cfg, pos, 1000.0, 500.0)
    assert np.max(np.abs(nxt - (p64 - 0.5 * cfg.astype(np.float64)))) <= 2e-5


@pytest.mark.parametrize("scale,rescale", [(1.0, 0.0), (3.0, 0.0), (6.5, 0.7), (2.0, 1.0), (4.0, -0.3)])
def test_cfg_closed_form(orc, scale, rescale):
    rng = np.random.default_rng(11)
    pos = rng.standard_normal((16, 3, 8, 10)).astype(np.float32)
    neg = (0.6 * pos + 0.5 * rng.standard_normal(pos.shape)).astype(np.float32)
    got = orc.apply_cfg(pos, neg, scale, rescale).astype(np.float64)
    p64, n64 = pos.astype(np.float64), neg.astype(np.float64)
    raw = n64 + scale * (p64 - n64)
    factor = 1.0 if rescale == 0.0 else rescale * np.std(p64, ddof=1) / np.std(raw, ddof=1) + (1 - rescale)
    np.testing.assert_allclose(got, raw * factor, rtol=2e-6, atol=2e-6)
    if rescale == 1.0:
        assert abs(np.std(got, ddof=1) - np.std(p64, ddof=1)) <= 1e-5 * np.std(p64, ddof=1)


def test_cfg_scale_zero_and_constant_output(orc):
    rng = np.random.default_rng(2)
    pos = rng.standard_normal(500).astype(np.float32)
    neg = rng.standard_normal(500).astype(np.float32)
    assert np.array_equal(orc.apply_cfg(pos, neg, 0.0, 0.0), neg)
    # a constant output has zero spread: the rescale is skipped (sampler.cpp:222)
    const = np.full(64, 0.5, np.float32)
    assert np.array_equal(orc.apply_cfg(pos[:64], const, 0.0, 0.9), const)
    # a single element has no spread either (count <= 1)
    assert np.array_equal(orc.apply_cfg(pos[:1], neg[:1], 2.0, 0.5), orc.apply_cfg(pos[:1], neg[:1], 2.0, 0.0))


def test_standard_deviation(orc):
    rng = np.random.default_rng(3)
    x = (3.0 + rng.standard_normal(10000)).astype(np.float32)
    assert abs(orc.standard_deviation(x) - np.std(x.astype(np.float64), ddof=1)) <= 1e-9
    assert orc.standard_deviation(x[:1]) == 0.0
    assert orc.standard_deviation(np.full(10, 7.0)) == 0.0


@pytest.mark.parametrize("t,t_next", [(1000.0, 750.0), (750.0, 500.0), (250.0, 0.0), (333.3, 123.4)])
def test_euler_step_closed_form(orc, t, t_next):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32)
    pred = rng.standard_normal(4096).astype(np.float32)
    got = orc.euler_step(pred, x, t, t_next).astype(np.float64)
    bt, bs = t / 1000.0, min(max(t_next / 1000.0, 0.0), 1.0)
    np.testing.assert_allclose(got, x + (bs - bt) * pred.astype(np.float64), rtol=0, atol=3e-6)


def test_euler_identities(orc):
    rng = np.random.default_rng(6)
    x = rng.standard_normal(2048).astype(np.float32)
    pred = rng.standard_normal(2048).astype(np.float32)
    for t in (1000.0, 600.0, 12.5):
        assert np.array_equal(orc.euler_endpoint(pred, x, t), orc.euler_step(pred, x, t, 0.0))
        assert np.array_equal(orc.euler_step(pred, x, t, 1500.0), orc.euler_step(pred, x, t, 1000.0))
        assert np.array_equal(orc.euler_step(pred, x, t, -20.0), orc.euler_step(pred, x, t, 0.0))
        np.testing.assert_allclose(orc.euler_step(pred, x, t, t), x, rtol=0, atol=2e-6)
    np.testing.assert_allclose(orc.euler_endpoint(pred, x, 400.0), x - 0.4 * pred.astype(np.float64),
                               rtol=0, atol=1e-6)


@pytest.mark.parametrize("steps", [-2, 0, 1, 4, 25, 50])
def test_timesteps(orc, steps):
    got = orc.euler_timesteps(steps)
    n = max(1, steps)
    assert got.shape == (n,)
    np.testing.assert_allclose(got, 1000.0 * (1.0 - np.arange(n) / n), rtol=0, atol=1e-4)
    assert got[0] == 1000.0
    if steps == 4:
        assert got.tolist() == [1000.0, 750.0, 500.0, 250.0]


def test_condition_ratio(orc):
    for s in (0.0, 0.05, 0.3, 1.0):
        # 256x256x37 pixels: shift 1, the ratio is the noise scale itself
        assert abs(orc.condition_ratio(s, 10, 32, 32) - s) <= 1e-6
        # 1280x720x145 pixels: shift 5
        assert abs(orc.condition_ratio(s, 37, 90, 160) - 5 * s / (1 + 4 * s)) <= 1e-6
    assert orc.condition_ratio(0.0, 21, 90, 160) == 0.0


def test_make_dit_input_channel_major(orc):
    rng = np.random.default_rng(7)
    lat = rng.standard_normal((16, 2, 4, 6)).astype(np.float32)
    cond = rng.standard_normal((16, 2, 4, 6)).astype(np.float32)
    got = orc.make_dit_input(lat, cond)
    expected = np.concatenate([lat, cond, np.ones((1, 2, 4, 6), np.float32)], axis=0)
    assert np.array_equal(got, expected)
    tok = orc.make_dit_input(lat.reshape(16, -1).T.copy(), cond.reshape(16, -1).T.copy(), channel_major=False)
    assert np.array_equal(tok, expected.reshape(33, -1).T)


# ---- host half of the library ABI (no device work) ------------------------

def test_abi_timesteps_and_ratio_match_oracle(hip, orc):
    for steps in (-1, 0, 1, 3, 7, 50):
        assert np.array_equal(hip.euler_timesteps(steps), orc.euler_timesteps(steps))
    for s, shape in ((0.0, (5, 8, 8)), (0.1, (21, 90, 160)), (0.25, (37, 90, 160)), (0.7, (3, 12, 20))):
        assert hip.condition_ratio(s, *shape) == orc.condition_ratio(s, *shape)


def test_abi_sampler_argument_errors(hip):
    lib = hip.load()
    fake = ctypes.c_void_p(0x1000)
    rc = lib.sv2_apply_cfg(fake, fake, fake, 10, 2.0, 0.5, None, 0, None)
    assert rc == hip.SV2_EINVAL and "workspace" in lib.sv2_last_error().decode()
    assert lib.sv2_apply_cfg(None, fake, fake, 10, 2.0, 0.0, None, 0, None) == hip.SV2_EINVAL
    assert lib.sv2_euler_step(fake, fake, fake, -1, 500.0, 250.0, None) == hip.SV2_EINVAL
    assert lib.sv2_euler_endpoint(fake, None, fake, 4, 500.0, None) == hip.SV2_EINVAL
    assert lib.sv2_make_condition(fake, fake, None, 4, 0.5, None) == hip.SV2_EINVAL
    assert lib.sv2_make_dit_input(None, fake, fake, 4, 1, None) == hip.SV2_EINVAL
    # empty inputs are a no-op, as the reference's loops over zero elements
    assert lib.sv2_euler_step(None, None, None, 0, 500.0, 250.0, None) == hip.SV2_OK
    assert lib.sv2_cfg_workspace_size(1 << 30) > 0
    assert lib.sv2_euler_timesteps(3, None) == hip.SV2_EINVAL
