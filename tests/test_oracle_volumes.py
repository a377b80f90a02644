"""Pins the volume oracle (oracle/volumes.py) by hand-worked cases and by what
the mathematics fixes: ratio tracking is an unbiased estimator of
exp(-density_scale * integral of the extinction along the chord), whatever
the (valid) majorant, and a majorant grid bounds every value a sampler can
read inside its cell.  CPU only."""
import math

import numpy as np

from oracle import render as OR
from oracle import volumes as V


def test_voxel_majorant_hand_case():
    # grid [D, H, W] = [2, 2, 2] with value 100 z + 10 y + x
    g = np.array([[[100 * z + 10 * y + x for x in range(2)] for y in range(2)] for z in range(2)], np.float32)
    x = np.array([[0.25, -0.75, 0.5]], np.float32)
    w = np.array([[1.0, 0.5, -2.0]], np.float32)
    # cell = trunc(((0.25, -0.75, 0.5) * 0.5 + 0.5) * 2) = (1, 0, 1); voxel [0,1] x [-1,0] x [0,1]
    # exits along w at t = 0.75, 1.5, 0.25
    m, d = V.voxel_majorant(g, x, w)
    assert m[0] == 101 and d[0] == np.float32(0.25)
    # a point outside the box clamps into the edge voxels; an axis-parallel ray exits on its own axis
    # (x outside the box: that axis's exit distances are +inf, as w is 0 along it)
    m, d = V.voxel_majorant(g, np.array([[-3.0, 0.5, 0.5]], np.float32), np.array([[0.0, 1.0, 0.0]], np.float32))
    assert m[0] == 110 and d[0] == np.float32(0.5)


def test_majorant_grid_hand_case():
    fine = np.array([1, 2, 3, 7, 0, 0, 4, 5], np.float32)[:, None]
    # linear: coarse cell 1 of 2 reads fine [3, 8) (pos 3.5 .. 7.5, one voxel past floor);
    # nearest: [4, 8)
    np.testing.assert_array_equal(V.majorant_grid(fine, [2], aligned=False, linear=True)[:, 0], [7, 7])
    np.testing.assert_array_equal(V.majorant_grid(fine, [2], aligned=False, linear=False)[:, 0], [7, 5])
    np.testing.assert_array_equal(V.majorant_grid(fine, [2], aligned=True, linear=False)[:, 0], [7, 5])
    np.testing.assert_array_equal(V.majorant_grid(fine, [1])[:, 0], [7])


def _sample(fine, t, aligned, linear):
    """A continuous-coordinate sampler of a 3-D grid [D, H, W] at t in [0, 1]^3
    (per dimension: pos = t (n - 1) aligned, t n - 0.5 otherwise; linear blends
    floor(pos) and floor(pos) + 1, nearest reads floor(pos + 0.5); clamped)."""
    idx, wts = [], []
    for d in range(3):
        n = fine.shape[d]
        pos = t[d] * (n - 1) if aligned else t[d] * n - 0.5
        if linear:
            i0 = math.floor(pos)
            f = pos - i0
            idx.append([min(max(i0, 0), n - 1), min(max(i0 + 1, 0), n - 1)])
            wts.append([1 - f, f])
        else:
            idx.append([min(max(math.floor(pos + 0.5), 0), n - 1)])
            wts.append([1.0])
    v = 0.0
    for a, wa in zip(idx[0], wts[0]):
        for b, wb in zip(idx[1], wts[1]):
            for c, wc in zip(idx[2], wts[2]):
                v += wa * wb * wc * fine[a, b, c]
    return v


def test_majorant_grid_bounds_every_sample():
    rng = np.random.default_rng(3)
    fine = rng.random((9, 7, 11)).astype(np.float32) ** 4
    for aligned in (False, True):
        for linear in (False, True):
            shape = [3, 2, 4]
            mg = V.majorant_grid(fine[..., None], shape, aligned, linear)[..., 0]
            for _ in range(600):
                cell = [int(rng.integers(s)) for s in shape]
                t = [(cell[d] + rng.random()) / shape[d] for d in range(3)]
                assert _sample(fine, t, aligned, linear) <= mg[tuple(cell)] + 1e-6
            # and it is the brute-force bound over the whole grid for one cell
            assert V.majorant_grid(fine[..., None], [1, 1, 1], aligned, linear)[0, 0, 0, 0] == fine.max()


def _chord_rays(n, rng):
    """Rays entering the box at x = -1 along +x (chord length 2)."""
    yz = rng.uniform(-0.9, 0.9, (n, 2))
    rays = np.zeros((n, 6), np.float32)
    rays[:, 0] = -2.0
    rays[:, 1:3] = yz
    rays[:, 3] = 1.0
    return rays


def _check_mean(T, expected):
    se = max(T.std(), 1e-3) / math.sqrt(T.size)
    assert abs(T.mean() - expected) < 5 * se, (T.mean(), expected, se)


def test_ratiotracking_unbiased_constant_extinction():
    rng = np.random.default_rng(0)
    rays = _chord_rays(20000, rng)
    sigma, ds = 0.7, 1.3
    ext = lambda p: np.full(p.shape[0], sigma, np.float32)  # noqa: E731
    expected = math.exp(-sigma * ds * 2.0)
    tight = V.ratiotracking(rays, ext, np.full((1, 1, 1), sigma, np.float32), [11, 22, 33, 44], density_scale=ds)
    assert set(np.unique(tight)) <= {0.0, 1.0}  # maj == sigma: the first collision zeroes T
    _check_mean(tight, expected)
    loose = V.ratiotracking(rays, ext, rng.uniform(sigma, 3 * sigma, (4, 4, 4)).astype(np.float32),
                            [55, 66, 77, 88], density_scale=ds)
    _check_mean(loose, expected)


def test_ratiotracking_unbiased_varying_extinction():
    # sigma(x) = a (x0 + 1): the optical depth of the chord is a * 2 * ds
    rng = np.random.default_rng(1)
    rays = _chord_rays(20000, rng)
    a, ds = 0.6, 0.9
    ext = lambda p: (np.float32(a) * (p[:, 0] + np.float32(1))).astype(np.float32)  # noqa: E731
    maj = np.empty((2, 2, 4), np.float32)
    maj[:] = (a * (np.arange(4) * 0.5 + 0.5) + 0.01)[None, None, :]  # per-x-slab max of sigma, a bit loose
    T = V.ratiotracking(rays, ext, maj, [9, 8, 7, 6], density_scale=ds)
    _check_mean(T, math.exp(-a * 2.0 * ds))


def test_ratiotracking_deterministic_cases():
    rng = np.random.default_rng(2)
    rays = _chord_rays(500, rng)
    zero = lambda p: np.zeros(p.shape[0], np.float32)  # noqa: E731
    np.testing.assert_array_equal(V.ratiotracking(rays, zero, np.ones((2, 2, 2), np.float32), [1, 2, 3, 4]), 1.0)
    miss = rays.copy()
    miss[:, 1] = 3.0  # parallel to the box, outside it
    one = lambda p: np.ones(p.shape[0], np.float32)  # noqa: E731
    np.testing.assert_array_equal(V.ratiotracking(miss, one, np.ones((1, 1, 1), np.float32), [1, 2, 3, 4]), 1.0)


def test_jittered_camera_rays():
    poses = np.array([[0.2, 0.1, -3.0, 0.0, 0.0, 0.0, 0.0, 1.0, 0.0]])
    centre = OR.camera_rays(5, 4, poses)
    np.testing.assert_array_equal(OR.camera_rays(5, 4, poses, jitter=np.full((1, 4, 5, 2), 0.5)), centre)
    # sub-pixel position (1, 1) of pixel (x, y) is position (0, 0) of pixel (x + 1, y + 1)
    ones = OR.camera_rays(5, 4, poses, jitter=np.ones((1, 4, 5, 2)))
    zeros = OR.camera_rays(5, 4, poses, jitter=np.zeros((1, 4, 5, 2)))
    np.testing.assert_allclose(ones[0, :-1, :-1], zeros[0, 1:, 1:], rtol=0, atol=1e-12)
