"""GPU parity of the Euler sampler and latent preparation (csrc/sampler.hip)
against the CPU oracle on identical seeded inputs:
  sv2_make_condition   make_condition_latent (engine.cpp:106-122)
  sv2_make_dit_input   make_dit_input (engine.cpp:125-149) and the token-major
                       layout of make_dit_input_vulkan (sampler.cpp:337-357)
  sv2_apply_cfg        EulerSampler::apply_cfg (sampler.cpp:201-236)
  sv2_euler_step       EulerSampler::step_to (sampler.cpp:239-265)
  sv2_euler_endpoint   EulerSampler::endpoint (sampler.cpp:267-285)

Bar: bit-identical to the oracle everywhere except the guidance rescale,
where the factor comes from double sums in another order: there every element
is within 2 fp32 ulps of the oracle's.  Shapes: the 720p x 21-frame latent
(16 x 6 x 90 x 160), element counts that are not a multiple of a workgroup,
one element, the reference's own 7-token runner case, and in-place updates.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

LATENT_720P = (16, 6, 90, 160)


@pytest.fixture(scope="module")
def sampler(hip):
    return hip.EulerSampler(4)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def within_ulps(gpu, ref, ulps=2):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    bound = ulps * np.spacing(np.maximum(np.abs(gpu), np.abs(ref)).astype(np.float32)).astype(np.float64)
    d = np.abs(gpu - ref)
    bad = d > bound
    assert not bad.any(), f"{int(bad.sum())} of {d.size} beyond {ulps} ulp, max diff {d.max():.3e}"


def pair(shape, seed, corr=0.6):
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(shape).astype(np.float32)
    b = (corr * a + 0.5 * rng.standard_normal(shape)).astype(np.float32)
    return a, b


@pytest.mark.parametrize("shape", [LATENT_720P, (16, 1, 3, 7), (1,)])
@pytest.mark.parametrize("ratio", [0.0, 0.25, 0.6818182])
def test_make_condition(sampler, orc, shape, ratio):
    enc, noise = pair(shape, 1)
    got = host(sampler.make_condition(dev(enc), dev(noise), ratio))
    assert np.array_equal(got, orc.make_condition(enc, noise, ratio))


@pytest.mark.parametrize("shape", [LATENT_720P, (16, 1, 5, 3)])
def test_make_dit_input(sampler, orc, shape):
    lat, cond = pair(shape, 2)
    got = host(sampler.make_dit_input(dev(lat), dev(cond)))
    assert np.array_equal(got, orc.make_dit_input(lat, cond))
    tl, tc = lat.reshape(16, -1).T.copy(), cond.reshape(16, -1).T.copy()
    got_t = host(sampler.make_dit_input(dev(tl), dev(tc), channel_major=False))
    assert np.array_equal(got_t, orc.make_dit_input(tl, tc, channel_major=False))


@pytest.mark.parametrize("shape", [LATENT_720P, (16, 1, 3, 7), (1,)])
@pytest.mark.parametrize("scale", [1.0, 5.0])
def test_cfg_plain(sampler, orc, shape, scale):
    pos, neg = pair(shape, 3)
    got = host(sampler.apply_cfg(dev(pos), dev(neg), scale, 0.0))
    assert np.array_equal(got, orc.apply_cfg(pos, neg, scale, 0.0))


@pytest.mark.parametrize("shape", [LATENT_720P, (16, 1, 3, 7), (2,), (1,)])
@pytest.mark.parametrize("scale,rescale", [(6.5, 0.7), (2.5, 0.4), (3.0, 1.0), (4.0, -0.3)])
def test_cfg_rescale(sampler, orc, shape, scale, rescale):
    pos, neg = pair(shape, 4)
    got = host(sampler.apply_cfg(dev(pos), dev(neg), scale, rescale))
    within_ulps(got, orc.apply_cfg(pos, neg, scale, rescale))


def test_cfg_rescale_constant_output_skips(sampler, orc):
    pos = np.random.default_rng(5).standard_normal(4097).astype(np.float32)
    const = np.full(4097, -0.75, np.float32)
    got = host(sampler.apply_cfg(dev(pos), dev(const), 0.0, 0.9))
    assert np.array_equal(got, const)
    assert np.array_equal(got, orc.apply_cfg(pos, const, 0.0, 0.9))


def test_reference_runner_case(sampler, orc):
    """tests/sampler_vulkan_runner.cpp:66-148 on the device: the 7-token
    [tokens, 16] pattern, condition ratio 0.25, CFG 2.5 / 0.4, step 1000 -> 500."""
    i = np.arange(16 * 7)
    pos = ((i % 13 - 6).astype(np.float32) * np.float32(0.07)).reshape(7, 16)
    neg = ((i % 9 - 4).astype(np.float32) * np.float32(0.05)).reshape(7, 16)
    p, n = dev(pos), dev(neg)
    cond = sampler.make_condition(p, n, 0.25)
    dit = sampler.make_dit_input(p, cond, channel_major=False)
    cfg = sampler.apply_cfg(p, n, 2.5, 0.4)
    nxt = sampler.step_to(cfg, p, 1000.0, 500.0)
    cond_h, dit_h, cfg_h, nxt_h = host(cond), host(dit), host(cfg), host(nxt)
    assert np.max(np.abs(cond_h - (0.75 * pos + 0.25 * neg))) <= 1e-6
    assert np.array_equal(dit_h[:, :16], pos) and np.array_equal(dit_h[:, 16:32], cond_h)
    assert np.all(dit_h[:, 32] == 1.0)
    within_ulps(cfg_h, orc.apply_cfg(pos, neg, 2.5, 0.4))
    assert np.max(np.abs(nxt_h - (pos - 0.5 * cfg_h))) <= 2e-5
    assert np.array_equal(nxt_h, orc.euler_step(cfg_h, pos, 1000.0, 500.0))


@pytest.mark.parametrize("t,t_next", [(1000.0, 750.0), (500.0, 250.0), (333.3, 123.4), (900.0, 1500.0),
                                      (100.0, -5.0)])
@pytest.mark.parametrize("shape", [LATENT_720P, (3, 1, 1, 333)])
def test_euler_step(sampler, orc, t, t_next, shape):
    pred, x = pair(shape, 6, corr=0.0)
    got = host(sampler.step_to(dev(pred), dev(x), t, t_next))
    assert np.array_equal(got, orc.euler_step(pred, x, t, t_next))


@pytest.mark.parametrize("t", [1000.0, 250.0, 12.5])
def test_euler_endpoint(sampler, orc, t):
    pred, x = pair(LATENT_720P, 7, corr=0.0)
    got = host(sampler.endpoint(dev(pred), dev(x), t))
    assert np.array_equal(got, orc.euler_endpoint(pred, x, t))


def test_in_place_updates(sampler, orc):
    pos, neg = pair((16, 2, 10, 12), 8)
    pred, x = pair((16, 2, 10, 12), 9, corr=0.0)
    p = dev(pos)
    sampler.apply_cfg(p, dev(neg), 4.0, 0.5, output=p)
    within_ulps(host(p), orc.apply_cfg(pos, neg, 4.0, 0.5))
    xd = dev(x)
    sampler.step_to(dev(pred), xd, 750.0, 500.0, output=xd)
    assert np.array_equal(host(xd), orc.euler_step(pred, x, 750.0, 500.0))


@pytest.mark.parametrize("rescale", [0.0, 0.7])
def test_sampler_loop(hip, orc, rescale):
    """The engine loop's sampler half (engine.cpp:306-350) over 4 steps with
    fixed per-step predictions standing in for the two DiT calls: condition,
    33-channel input, CFG, Euler steps and the endpoint, all on one stream."""
    shape = (16, 2, 12, 16)
    rng = np.random.default_rng(10)
    latent = rng.standard_normal(shape).astype(np.float32)
    encoded = rng.standard_normal(shape).astype(np.float32)
    aug = rng.standard_normal(shape).astype(np.float32)
    preds = [pair(shape, 20 + k) for k in range(4)]
    ratio = hip.condition_ratio(0.1, *shape[1:])
    s = hip.EulerSampler(4)
    assert np.array_equal(s.timesteps, orc.euler_timesteps(4))

    cond_d = s.make_condition(dev(encoded), dev(aug), ratio)
    lat_d = dev(latent)
    cond = orc.make_condition(encoded, aug, ratio)
    lat = latent
    ts = s.timesteps
    for k, t in enumerate(ts):
        dit_d = s.make_dit_input(lat_d, cond_d)
        dit = orc.make_dit_input(lat, cond)
        assert np.array_equal(host(dit_d), dit)
        pos, neg = preds[k]
        guided_d = s.apply_cfg(dev(pos), dev(neg), 6.5, rescale)
        guided = orc.apply_cfg(pos, neg, 6.5, rescale)
        g_h = host(guided_d)
        if rescale == 0.0:
            assert np.array_equal(g_h, guided)
        else:
            within_ulps(g_h, guided)
        # continue both sides from the device's guided prediction so that the
        # step comparison stays bit-exact
        if k + 1 < len(ts):
            lat_d = s.step_to(guided_d, lat_d, float(t), float(ts[k + 1]))
            lat = orc.euler_step(g_h, lat, float(t), float(ts[k + 1]))
        else:
            lat_d = s.endpoint(guided_d, lat_d, float(t))
            lat = orc.euler_endpoint(g_h, lat, float(t))
        assert np.array_equal(host(lat_d), lat)
