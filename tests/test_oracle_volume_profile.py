"""Pins of oracle.volumes.volume_profile and its helpers (VolumeProfile,
src/rdv/domain/volumes.py:503-550, shaders/volumes/volume_profile.h:1-167) by
what the mathematics fixes:
  * crossing_tau is the mean of a unit-rate exponential truncated to
    [0, scale * tau] (numerical integration), 0.5 x below 0.01 and 1 past 20;
  * ortho_basis gives an orthonormal right-handed frame (t0 x t1 = n);
  * hg_sample is the Henyey-Greenstein distribution: unit vectors whose mean
    cosine with w is g (and E[cos^2] = 1/3 at g = 0), with cos(theta)'s CDF
    matching the closed form (Kolmogorov-Smirnov);
  * a constant medium (extinction sigma, majorant sigma) fixes every output:
    tau = the fp32 sum of sigma * ds * step over the march's step count, the
    depth index where ctau * scale first reaches the crossing value, the light
    ray's raymarched transmittance exp(-sigma' step m), and ratio tracking with
    a tight majorant is 0 or 1 with mean exp(-sigma' L) along each sampled
    direction;
  * misses and an empty medium give the documented zeros.
A planted mistake in the crossing formula is caught."""
import math

import numpy as np
import pytest

from oracle import random as RNG
from oracle import volumes as V

F = np.float32


def _truncated_exp_mean(x: float) -> float:
    from scipy.integrate import quad
    num, _ = quad(lambda t: t * math.exp(-t), 0.0, x)
    den, _ = quad(lambda t: math.exp(-t), 0.0, x)
    return num / den


@pytest.mark.parametrize("scale,tau", [(0.1, 0.2), (0.5, 1.0), (0.9, 3.0), (1.0, 7.5), (0.3, 60.0), (1.0, 19.9)])
def test_crossing_tau_is_truncated_exponential_mean(scale, tau):
    x = scale * tau
    want = _truncated_exp_mean(x) if x <= 20 else 1.0
    assert abs(float(V.crossing_tau(scale, tau)) - want) < 2e-5 * max(1.0, want)


def test_crossing_tau_small_and_large():
    for x in (1e-4, 3e-3, 0.0099):
        assert float(V.crossing_tau(1.0, x)) == pytest.approx(0.5 * x, rel=1e-6)
        # the truncated mean itself tends to x / 2
        assert _truncated_exp_mean(x) == pytest.approx(0.5 * x, rel=0.01)
    assert float(V.crossing_tau(1.0, 20.5)) == 1.0


def test_planted_crossing_mistake_is_caught():
    def wrong(scale, tau):  # a sign slip in the denominator
        x = F(scale) * F(tau)
        return F(1) - F(x * np.exp(-x)) / F(1 + np.exp(-x))
    assert abs(float(wrong(0.5, 1.0)) - _truncated_exp_mean(0.5)) > 1e-3


def test_ortho_basis_is_orthonormal_and_right_handed():
    rng = np.random.default_rng(0)
    for _ in range(200):
        n = rng.normal(size=3)
        n = (n / np.linalg.norm(n)).astype(F)
        t0, t1 = V.ortho_basis(n)
        M = np.stack([t0, t1, n]).astype(np.float64)
        np.testing.assert_allclose(M @ M.T, np.eye(3), atol=2e-6)
        np.testing.assert_allclose(np.cross(t0, t1), n, atol=2e-6)


@pytest.mark.parametrize("g", [0.0, 0.3, -0.6, 0.85])
def test_hg_sample_distribution(g):
    rng = np.random.default_rng(1)
    w = rng.normal(size=3)
    w = (w / np.linalg.norm(w)).astype(F)
    st = RNG.spawn((11, 22, 33, 44), np.arange(1))
    cos = []
    for _ in range(6000):
        d, st = V.hg_sample(w, g, st)
        assert abs(np.linalg.norm(d.astype(np.float64)) - 1) < 1e-5
        cos.append(float(np.dot(d.astype(np.float64), w)))
    cos = np.array(cos)
    se = cos.std() / math.sqrt(cos.size)
    assert abs(cos.mean() - g) < 5 * se + 1e-3
    if g == 0.0:
        assert abs((cos ** 2).mean() - 1 / 3) < 0.02
    # CDF of cos(theta) for Henyey-Greenstein
    def cdf(mu):
        if abs(g) < 1e-3:
            return (mu + 1) / 2
        return (1 - g * g) / (2 * g) * (1 / np.sqrt(1 + g * g - 2 * g * mu) - 1 / (1 + g))
    xs = np.sort(cos)
    emp = np.arange(1, xs.size + 1) / xs.size
    assert np.max(np.abs(emp - cdf(xs))) < 1.63 / math.sqrt(xs.size)  # KS at 1%


def _rays_along_z(n, seed, spread=0.6):
    g = np.random.default_rng(seed)
    o = np.zeros((n, 3))
    o[:, :2] = g.uniform(-spread, spread, (n, 2))
    o[:, 2] = -3.0
    w = np.tile([0.0, 0.0, 1.0], (n, 1))
    return np.concatenate([o, w], 1).astype(F)


def _const(sigma):
    return lambda p: np.full(p.shape[0], sigma, F)


def test_constant_medium_closed_forms():
    sigma, ds, step, g = F(1.25), 1.5, 0.01, 0.4
    rays = _rays_along_z(12, 0)
    grid = np.full((4, 4, 4), sigma, F)
    thr = [0.9, 0.5, 0.2]
    r = V.volume_profile(rays, _const(sigma), grid, (3, 1, 4, 1), thr, 3, environment_samples=0, g=g,
                         step_size=step, density_scale=ds, light_direction=(0.0, 1.0, 0.0))
    out = r["out"]
    assert r["valid"].all()
    DS = len(thr)
    inc = F(F(sigma * F(ds)) * F(step))
    for i in range(rays.shape[0]):
        # entry at t = 2 (z = -1), exit at t = 4; march count by an independent loop
        t, n = F(2.0), 0
        while t < F(4.0):
            n += 1
            t = F(t + F(step))
        tau = F(0)
        for _ in range(n):
            tau = F(tau + inc)
        assert abs(float(tau) - float(sigma) * ds * step * n) < 1e-4
        S = 1 - math.exp(-float(tau))
        assert out[i, -1] == pytest.approx(S, rel=1e-6)
        # first depth: the first k with (k + 1) inc * scale >= crossing
        tc = _truncated_exp_mean(thr[0] * float(tau))
        k = math.ceil(tc / (thr[0] * float(inc))) - 1
        t0 = 2.0 + k * step
        assert 1.0 / out[i, 0] - 0.1 == pytest.approx(t0, abs=1.5 * step)
        # light ray: +y from the sample position (y0 + ...), exit at y = 1
        y0 = rays[i, 1]
        m = math.ceil((1.0 - y0) / step)
        nee_ds = (0.2 + 0.8 * (1 - g)) * ds
        Tl = math.exp(-float(sigma) * nee_ds * step * m)
        assert out[i, DS + 1] / out[i, -1] == pytest.approx(Tl, rel=2e-3)
        assert out[i, DS] == pytest.approx(0.2 * math.log(1 + float(tau)), rel=1e-6)
        assert out[i, DS + 2 + 2 * 3] == F(g)


def test_tight_majorant_ratio_tracking_mean():
    sigma, ds, g = F(0.9), 1.0, 0.0
    rays = _rays_along_z(150, 1, spread=0.3)
    grid = np.full((2, 2, 2), sigma, F)
    r = V.volume_profile(rays, _const(sigma), grid, (9, 8, 7, 6), [0.5], 1, environment_samples=16, g=g,
                         step_size=0.02, density_scale=ds)
    wts, dirs, spos, S = r["wts"], r["dirs"], r["spos"], r["out"][:, -1]
    T = wts / S[:, None]
    assert set(np.unique(np.round(T, 5))) <= {0.0, 1.0}
    nee_ds = (0.2 + 0.8 * (1 - g)) * ds
    # exit distance of each sampled direction from the sample position
    from oracle.render import ray_box32
    L = ray_box32(np.repeat(spos, 16, 0), dirs.reshape(-1, 3))[1].reshape(T.shape)
    expect = np.exp(-float(sigma) * nee_ds * L)
    se = np.sqrt((expect * (1 - expect)).sum()) / T.size
    assert abs(T.mean() - expect.mean()) < 5 * se


def test_miss_and_empty_medium():
    rays = np.array([[0.0, 3.0, -3.0, 0.0, 0.0, 1.0],   # misses the box
                     [0.0, 0.0, -3.0, 0.0, 0.0, 1.0]], F)  # meets it, empty medium
    grid = np.zeros((3, 3, 3), F)
    r = V.volume_profile(rays, _const(0.0), grid, (1, 2, 3, 4), [0.3, 0.6], 2, environment_samples=2,
                         albedo=lambda p: np.full((p.shape[0], 2), 0.5, F),
                         environment=lambda w: np.ones((w.shape[0], 2), F))
    assert not r["out"].any()
    assert not r["valid"].any()


def test_sample_index_and_reencoding():
    sigma = F(2.0)
    rays = _rays_along_z(3, 2)
    grid = np.full((1, 1, 1), sigma, F)
    thr = [0.95, 0.6, 0.3, 0.1]
    a = V.volume_profile(rays, _const(sigma), grid, (1, 1, 1, 1), thr, 1, environment_samples=0, step_size=0.005)
    b = V.volume_profile(rays, _const(sigma), grid, (1, 1, 1, 1), thr, 1, environment_samples=0, step_size=0.005,
                         sample_index=2)
    # the sample position moves to depth 2's t along the ray
    t0 = 1.0 / a["out"][:, 0] - 0.1
    np.testing.assert_allclose(a["spos"][:, 2], rays[:, 2] + t0, atol=1e-5)
    assert (b["spos"][:, 2] >= a["spos"][:, 2]).all()
    # re-encoding: out[i] = 1 / (1 + 10 sqrt(t_i - t_{i-1})) is in (0, 1]
    assert ((a["out"][:, 1:4] > 0) & (a["out"][:, 1:4] <= 1)).all()
