"""Pins oracle/render.py: camera geometry, the slab test, compositing and the
transmittance march against closed forms and brute force (CPU only)."""
import math

import numpy as np
import pytest

from oracle import render as R

POSE = np.array([[0.0, 0.0, -3.5, 0.0, 0.0, 0.0, 0.0, 1.0, 0.0]])


def _const_field(sigma_logit: float, rgb_logits, width: int = 64, out: int = 4):
    """3 -> 64 -> 64 -> 64 -> out with zero weights: the head returns its bias."""
    layers = [(np.zeros((width, 3), np.float32), np.zeros(width, np.float32)),
              (np.zeros((width, width), np.float32), np.zeros(width, np.float32)),
              (np.zeros((width, width), np.float32), np.zeros(width, np.float32))]
    b = np.array([sigma_logit] + list(rgb_logits), np.float32)[:out]
    layers.append((np.zeros((out, width), np.float32), b))
    return layers


def test_single_pixel_camera_looks_at_target():
    r = R.camera_rays(1, 1, POSE)
    np.testing.assert_allclose(r[0, 0, 0], [0, 0, -3.5, 0, 0, 1], atol=1e-15)
    pose = np.array([[1.0, 2.0, 3.0, -2.0, 0.5, 1.0, 0.0, 0.0, 1.0]])
    d = pose[0, 3:6] - pose[0, 0:3]
    np.testing.assert_allclose(R.camera_rays(1, 1, pose)[0, 0, 0, 3:], d / np.linalg.norm(d), atol=1e-15)


def test_camera_ray_angles_match_the_pinhole_model():
    """cos(angle to the view axis) = sz / |(sx, sy, sz)| with s = (p.x aspect, p.y, 1 / tan(fov / 2))."""
    W, H, fov = 6, 4, 0.9
    r = R.camera_rays(W, H, POSE, fov=fov)
    px = (np.arange(W) + 0.5) / W * 2 - 1
    py = (np.arange(H) + 0.5) / H * 2 - 1
    sz = 1 / math.tan(fov / 2)
    sx, sy = np.meshgrid(px * (W / H), py)
    want = sz / np.sqrt(sx ** 2 + sy ** 2 + sz ** 2)
    np.testing.assert_allclose(r[0, :, :, 5], want, atol=1e-14)  # view axis is +z here
    # +x image axis is cross(up, z) = (+1, 0, 0) for up = +y, z = +z; +y image axis is +y
    assert np.all(np.diff(r[0, 0, :, 3]) > 0) and np.all(np.diff(r[0, :, 0, 4]) > 0)
    np.testing.assert_allclose(np.linalg.norm(r[..., 3:], axis=-1), 1.0, atol=1e-15)


def test_ray_box_closed_forms():
    x = np.array([[0.0, 0.0, -3.5], [0.2, -0.3, 0.1], [3.0, 3.0, -3.5]])
    w = np.array([[0.0, 0.0, 1.0], [0.0, 0.0, 1.0], [0.0, 0.0, 1.0]])
    tmin, tmax = R.ray_box(x + 1e-300, w + np.array([1e-300, 1e-300, 0]))
    np.testing.assert_allclose(tmin[:2], [2.5, -1.1], atol=1e-12)
    np.testing.assert_allclose(tmax[:2], [4.5, 0.9], atol=1e-12)
    assert tmin[2] > tmax[2]  # misses the box
    t32 = R.ray_box32(x[:2] + np.float32(1e-20), w[:2] + np.array([1e-20, 1e-20, 0]))
    np.testing.assert_allclose(t32[0], [2.5, -1.1], atol=1e-6)


def test_composite_constant_medium_closed_form():
    S, sig, L = 128, 0.7, 2.0
    c = np.array([0.2, 0.5, 0.9])
    s = np.zeros((1, S, 4))
    s[..., 0], s[..., 1:] = sig, c
    np.testing.assert_allclose(R.composite(s, np.array([L / S])), [c * (1 - math.exp(-sig * L))], rtol=1e-12)


def test_composite_matches_sequential_loop():
    rng = np.random.default_rng(0)
    s = rng.uniform(0, 3, (5, 17, 4))
    dt = rng.uniform(0.001, 0.3, 5)
    want = np.zeros((5, 3))
    for r in range(5):
        T = 1.0
        for i in range(17):
            a = 1 - math.exp(-s[r, i, 0] * dt[r])
            want[r] += T * a * s[r, i, 1:]
            T *= 1 - a
    np.testing.assert_allclose(R.composite(s, dt), want, rtol=1e-12)


def test_render_ea_constant_field_closed_form():
    """sigma, c constant: C = c (1 - exp(-sigma L)) with L the chord through the box."""
    layers = _const_field(0.3, [-0.5, 0.25, 1.5])
    rays = R.camera_rays(5, 3, POSE).reshape(-1, 6)
    got = R.render_ea(rays, layers, 64)
    tmin, tmax = R.ray_box(rays[:, :3], rays[:, 3:])
    hit = ~((tmax <= 0) | (tmin > tmax))
    assert hit.sum() >= 5 and (~hit).sum() >= 2
    L = np.where(hit, tmax - np.maximum(tmin, 0), 0.0)
    # the head returns its fp32 bias (zero weights): sigma = softplus(0.3), c = sigmoid(logits)
    b = np.array([0.3, -0.5, 0.25, 1.5], np.float32).astype(np.float64)
    sigma = math.log1p(math.exp(b[0]))
    c = 1 / (1 + np.exp(-b[1:]))
    want = c[None, :] * (1 - np.exp(-sigma * L))[:, None]
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-15)


def _fp32_march_count(d: np.float32, step: np.float32) -> int:
    n = 0
    while d > 0 and n < 4096:
        d = np.float32(d - step)
        n += 1
    return n


def test_transmittance_constant_extinction_closed_form():
    layers = _const_field(0.4, [], out=1)
    rays = R.camera_rays(4, 4, POSE).reshape(-1, 6).astype(np.float32)
    got = R.raymarch_transmittance(rays, layers, head="softplus", step=0.002)
    sigma = np.float32(math.log1p(math.exp(0.4)))
    x, w = rays[:, :3], rays[:, 3:]
    tmin, tmax = R.ray_box32(x, w)
    for i in range(rays.shape[0]):
        t0 = max(np.float32(0), tmin[i])
        n = _fp32_march_count(np.float32(tmax[i] - t0), np.float32(0.002))
        assert abs(got[i] - math.exp(-float(sigma) * 0.002 * n)) < 2e-5 * math.exp(-float(sigma) * 0.002 * n)


def test_transmittance_cutoff_and_miss():
    layers = _const_field(12.0, [], out=1)  # sigma ~ 12: tau passes 16 after ~667 steps of 0.002
    rays = np.array([[0, 0, -3.5, 0, 0, 1], [0, 0, -3.5, 0, 0.6, 0.8]], np.float32)
    got = R.raymarch_transmittance(rays, layers, head="softplus", step=0.002)
    assert got[0] == 0.0      # 2.0 long chord: tau ~ 24 > 16
    assert got[1] == 1.0      # leaves the y slab (t = 1.67) before entering the z slab (t = 3.125)


def test_planted_mistake_is_caught(monkeypatch):
    """An inclusive transmittance (T_i counting sample i itself) breaks the closed form."""
    def bad(sigma_rgb, dt):
        s = np.asarray(sigma_rgb, np.float64)
        a = s[..., 0] * dt[:, None]
        T = np.cumprod(np.exp(-a), axis=1)
        return np.sum((T * (1 - np.exp(-a)))[..., None] * s[..., 1:4], axis=1)
    monkeypatch.setattr(R, "composite", bad)
    S, sig, L = 128, 0.7, 2.0
    s = np.zeros((1, S, 4))
    s[..., 0], s[..., 1:] = sig, 0.5
    assert abs(R.composite(s, np.array([L / S]))[0, 0] - 0.5 * (1 - math.exp(-sig * L))) > 1e-3
