"""Pins of the oracle's VolumeProfileDDA march (oracle/volumes.py dda_march_ts,
volume_profile(dda_grid=...)) against an independent construction: the cells a
ray crosses from the sorted crossings of the grid planes (float64), each cell
marched from its entry in fixed steps."""
import math

import numpy as np
import pytest

from oracle import volumes as V

F = np.float32


def _segments(x, wo, tmin, tmax, dims):
    """Cells crossed by x + wo t, t in [tmin, tmax): [(t0, t1, (cx, cy, cz))] from
    the sorted plane crossings (float64), the cell of each segment by its midpoint."""
    x = np.asarray(x, np.float64)
    wo = np.asarray(wo, np.float64)
    cuts = {float(tmin), float(tmax)}
    for i in range(3):
        if wo[i] == 0:
            continue
        for k in range(dims[i] + 1):
            t = (-1.0 + 2.0 * k / dims[i] - x[i]) / wo[i]
            if tmin < t < tmax:
                cuts.add(t)
    ts = sorted(cuts)
    segs = []
    for a, b in zip(ts[:-1], ts[1:]):
        if b - a < 1e-6:  # float64 crossings within float32 rounding of tmin / tmax
            continue
        m = x + wo * (0.5 * (a + b))
        c = tuple(min(max(int(math.floor((m[i] + 1.0) * 0.5 * dims[i])), 0), dims[i] - 1) for i in range(3))
        segs.append((a, b, c))
    return segs


def _expected(x, wo, tmin, tmax, step, grid):
    D, H, W = grid.shape
    out = []
    for a, b, c in _segments(x, wo, tmin, tmax, (W, H, D)):
        if grid[c[2], c[1], c[0]] > 0:
            n = math.ceil((b - a) / step)
            out.append((a, n))
    return out


def _ray(rng):
    o = rng.uniform(-0.9, 0.9, 3).astype(F)
    w = rng.normal(size=3)
    w = (w / np.linalg.norm(w)).astype(F)
    tmin, tmax = V._box(o, w)
    return o, w, max(F(0), tmin), tmax


@pytest.mark.parametrize("seed", range(6))
def test_dda_samples_each_crossed_cell_from_its_entry(seed):
    rng = np.random.default_rng(seed)
    grid = np.ones((3, 5, 4), F)
    x, w, tmin, tmax = _ray(rng)
    step = F(0.0137)
    ts = V.dda_march_ts(x, w, tmin, tmax, step, grid)
    exp = _expected(x, w, tmin, tmax, float(step), grid)
    assert ts.size == sum(n for _, n in exp)
    k = 0
    for a, n in exp:  # each marched cell starts at its entry, then steps of `step`
        assert abs(float(ts[k]) - a) < 2e-5
        if n > 1:
            assert abs(float(ts[k + 1]) - float(ts[k]) - float(step)) < 2e-6
        k += n


@pytest.mark.parametrize("seed", range(4))
def test_dda_skips_empty_cells(seed):
    rng = np.random.default_rng(10 + seed)
    grid = (rng.uniform(size=(4, 4, 4)) > 0.5).astype(F)
    x, w, tmin, tmax = _ray(rng)
    step = F(0.011)
    ts = V.dda_march_ts(x, w, tmin, tmax, step, grid)
    exp = _expected(x, w, tmin, tmax, float(step), grid)
    assert ts.size == sum(n for _, n in exp)
    for t in ts:  # every sample lies in a cell whose value is > 0 (just after t: t may sit on an entry)
        p = x.astype(np.float64) + w.astype(np.float64) * (float(t) + 1e-6)
        c = [min(max(int(math.floor((p[i] + 1) * 0.5 * 4)), 0), 3) for i in range(3)]
        assert grid[c[2], c[1], c[0]] > 0


@pytest.mark.parametrize("axis", [0, 1, 2])
def test_dda_zero_direction_component(axis):
    """A direction parallel to one axis' planes: that axis never comes first, and
    the walk matches the plane crossings of the other two (finite sample times)."""
    rng = np.random.default_rng(40 + axis)
    grid = np.ones((4, 3, 5), F)
    for _ in range(4):
        x = rng.uniform(-0.9, 0.9, 3).astype(F)
        w = rng.normal(size=3)
        w[axis] = 0.0
        w = (w / np.linalg.norm(w)).astype(F)
        tmin, tmax = V._box(x, w)
        tmin = max(F(0), tmin)
        step = F(0.013)
        ts = V.dda_march_ts(x, w, tmin, tmax, step, grid)
        assert np.isfinite(ts).all()
        assert ts.size == sum(n for _, n in _expected(x, w, tmin, tmax, float(step), grid))


def test_planted_march_without_reanchoring_is_caught():
    """A march that ignores the cell exits (VolumeProfile's plain march over the
    same interval) fails the per-cell count on a ray that crosses several cells."""
    grid = np.ones((3, 5, 4), F)
    x = np.array([-0.95, -0.9, -0.85], F)  # a diagonal through many cells
    w = np.array([1.0, 0.9, 0.8], F)
    w = (w / np.linalg.norm(w)).astype(F)
    tmin, tmax = V._box(x, w)
    tmin = max(F(0), tmin)
    step = F(0.0137)
    exp = _expected(x, w, tmin, tmax, float(step), grid)
    assert len(exp) > 5
    assert V.dda_march_ts(x, w, tmin, tmax, step, grid).size == sum(n for _, n in exp)
    plain = V._march_ts(tmin, tmax, step, V.MAX_MARCH)
    assert plain.size != sum(n for _, n in exp)


def test_constant_medium_profile_closed_form():
    """A grid of ones and a constant extinction: tau = sigma * ds * step * N
    (float32 sums), with N the DDA's sample count; S and 0.2 log(1 + tau) follow."""
    rng = np.random.default_rng(7)
    grid = np.ones((2, 3, 2), F)
    rays = []
    for _ in range(5):
        x, w, _, _ = _ray(rng)
        rays.append(np.concatenate([x - 2.5 * w, w]))  # from outside the box
    rays = np.array(rays, F)
    sigma, ds, step = 0.7, 1.3, 0.01
    res = V.volume_profile(rays, lambda p: np.full(p.shape[0], sigma, F), grid, (1, 2, 3, 4), [0.9, 0.5], 1,
                           environment_samples=0, step_size=step, density_scale=ds, dda_grid=grid,
                           albedo=lambda p: np.full((p.shape[0], 1), 0.5, F),
                           environment=lambda d: np.ones((d.shape[0], 1), F))
    for i, r in enumerate(rays):
        x, w = r[:3], r[3:]
        tmin, tmax = V._box(x, w)
        tmin = max(F(0), tmin)
        n = V.dda_march_ts(x, w, tmin, tmax, F(step), grid).size
        inc = F(F(F(sigma) * F(ds)) * F(step))
        tau = F(0)
        for _ in range(n):
            tau = F(tau + inc)
        out = res["out"][i]
        assert out[-1] == F(F(1) - F(np.exp(F(-tau))))
        if res["valid"][i]:
            assert out[2] == F(F(0.2) * F(np.log(F(F(1) + tau))))


def test_empty_grid_gives_no_depth():
    rays = np.array([[0.1, 0.2, -3.0, 0.0, 0.0, 1.0]], F)
    grid = np.zeros((2, 2, 2), F)
    res = V.volume_profile(rays, lambda p: np.full(p.shape[0], 5.0, F), np.ones((2, 2, 2), F), (1, 2, 3, 4),
                           [0.5], 1, environment_samples=0, dda_grid=grid,
                           albedo=lambda p: np.full((p.shape[0], 1), 0.5, F),
                           environment=lambda d: np.ones((d.shape[0], 1), F))
    assert res["valid"][0] == 0 and res["out"][0, -1] == 0  # tau = 0: S = 0, no depth
