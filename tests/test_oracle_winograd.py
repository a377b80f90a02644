"""Pins oracle/winograd.py: scalar golden vectors, the F(2x2,3x3) identity,
closed forms and a planted mistake (CPU only)."""
import glob
import os

import numpy as np
import pytest
import torch

from oracle import winograd as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
SHAPES = [(6, 8, 5, 16), (4, 4, 64, 32), (10, 6, 17, 48), (2, 2, 1, 16)]


def _case(H, W, C, K, seed=0):
    rng = np.random.default_rng(seed)
    return rng.uniform(-1, 1, (H, W, C)), rng.normal(0, 0.1, (3, 3, C, K)), rng.normal(0, 1, K)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "winograd_*.npz"))))
def test_oracle_matches_scalar_golden(path):
    z = np.load(path, allow_pickle=False)
    np.testing.assert_array_equal(O.transform_weight(z["w"]), z["U"])
    # same fp32 operation order everywhere; M is rounded once from an exact sum in both
    np.testing.assert_array_equal(O.winograd_conv(z["x"], z["w"], z["b"]), z["y"])


@pytest.mark.parametrize("H,W,C,K", SHAPES)
def test_exact_winograd_equals_direct_conv(H, W, C, K):
    """A^T[(G g G^T) * (B^T d B)]A is the 3x3 correlation: pins G, B^T, A^T and the patch indexing."""
    x, w, b = _case(H, W, C, K)
    np.testing.assert_allclose(O.winograd_conv(x, w, b, exact=True), O.direct_conv(x, w, b), rtol=0, atol=1e-12)


@pytest.mark.parametrize("H,W,C,K", SHAPES[:3])
def test_direct_conv_equals_torch_conv2d(H, W, C, K):
    x, w, b = _case(H, W, C, K, seed=1)
    t = torch.nn.functional.conv2d(torch.tensor(x).permute(2, 0, 1)[None], torch.tensor(w).permute(3, 2, 0, 1),
                                   torch.tensor(b), padding=1)[0].permute(1, 2, 0).numpy()
    np.testing.assert_allclose(O.direct_conv(x, w, b), t, rtol=0, atol=1e-12)


def test_identity_filter_returns_input():
    """w[1][1][c][c] = 1: y = x (x on a grid of eighths, so every rounding is exact)."""
    rng = np.random.default_rng(2)
    C = 16
    x = rng.integers(-16, 17, (8, 6, C)) / 8.0
    w = np.zeros((3, 3, C, C))
    w[1, 1] = np.eye(C)
    np.testing.assert_array_equal(O.winograd_conv(x, w), x)
    np.testing.assert_array_equal(O.direct_conv(x, w), x)


def test_shift_filter_moves_image():
    """A tap at (r, s) = (0, 2) reads x[h - 1][w + 1] (zero outside): checks orientation and padding."""
    rng = np.random.default_rng(3)
    x = rng.integers(-16, 17, (6, 8, 1)) / 8.0
    w = np.zeros((3, 3, 1, 16))
    w[0, 2, 0, :] = 1.0
    y = O.winograd_conv(x, w)
    want = np.zeros((6, 8))
    want[1:, :-1] = x[:-1, 1:, 0]
    for k in range(16):
        np.testing.assert_array_equal(y[:, :, k], want)


@pytest.mark.parametrize("r,s", [(0, 0), (1, 1), (2, 1), (0, 2)])
def test_transform_weight_of_a_delta_is_an_outer_product(r, s):
    w = np.zeros((3, 3, 1, 1))
    w[r, s, 0, 0] = 1.0
    U = O.transform_weight(w)[:, 0, 0].reshape(4, 4)
    np.testing.assert_array_equal(U, np.outer(O.G[:, r], O.G[:, s]))


def test_transforms_are_exact_on_small_integers():
    rng = np.random.default_rng(4)
    d = rng.integers(-8, 9, (50, 4, 4)).astype(np.float64)
    np.testing.assert_array_equal(O.winograd_fwd_f32(d), O.BT @ d @ O.BT.T)
    M = rng.integers(-100, 101, (50, 4, 4)).astype(np.float64)
    np.testing.assert_array_equal(O.winograd_inv_f32(M), O.AT @ M @ O.AT.T)


def test_fp16_path_within_stated_tolerance_of_direct():
    """Benchmark-shaped statistics (x in [0,1], w ~ N(0, sqrt(2/576)), 64 -> 64, ReLU) on a
    64x64 crop: the fp16-operand path stays within |e| <= 2e-3 max(1, max|y|) + 1e-2 |y|."""
    rng = np.random.default_rng(5)
    x = O.f16(rng.uniform(0, 1, (64, 64, 64)))
    w = O.f16(rng.normal(0, np.sqrt(2 / 576), (3, 3, 64, 64)))
    got = O.winograd_conv(x, w, relu=True)
    ref = O.direct_conv(x, w, relu=True)
    assert np.all(np.abs(got - ref) <= 2e-3 * max(1.0, np.abs(ref).max()) + 1e-2 * np.abs(ref))


def test_planted_mistake_is_caught(monkeypatch):
    """Transposing B^T in the oracle breaks the identity check above."""
    x, w, b = _case(4, 6, 3, 16)
    monkeypatch.setattr(O, "BT", O.BT.T.copy())
    assert np.abs(O.winograd_conv(x, w, b, exact=True) - O.direct_conv(x, w, b)).max() > 1e-3
