"""Pins oracle/mlp.py: golden scalar vectors, closed forms and invariants (CPU only)."""
import glob
import os

import numpy as np
import pytest

from oracle import mlp as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _load_chain(path):
    z = np.load(path, allow_pickle=False)
    dims = list(z["dims"])
    layers = [(z[f"W{i}"], z[f"b{i}"]) for i in range(len(dims) - 1)]
    return z["x"], layers, [str(a) for a in z["acts"]], [str(p) for p in z["precs"]], z["y"]


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "chain_*.npz"))))
def test_oracle_matches_scalar_golden(path):
    x, layers, acts, precs, y = _load_chain(path)
    got = O.mlp_forward(x, layers, acts, precs)
    # same arithmetic (exact sums, one fp32 rounding): equal up to a final-ulp tie
    np.testing.assert_allclose(got, y, rtol=2e-7, atol=1e-7)


def test_freq_encoding_matches_scalar_golden():
    z = np.load(os.path.join(GOLDEN, "freq_encoding.npz"), allow_pickle=False)
    got = O.freq_encode(z["p"], int(z["octaves"]))
    np.testing.assert_allclose(got, z["features"], atol=1e-6)


def test_freq_encoding_closed_forms():
    p = np.array([[0.0, 0.5, -0.25]], np.float32)
    f = O.freq_encode(p, 3, width=24)
    assert f.shape == (1, 24)
    np.testing.assert_array_equal(f[0, :3], p[0])
    # k = 0: sin(pi p), cos(pi p)
    np.testing.assert_allclose(f[0, 3:6], [0.0, 1.0, -np.sqrt(0.5)], atol=1e-7)
    np.testing.assert_allclose(f[0, 6:9], [1.0, 0.0, np.sqrt(0.5)], atol=1e-7)
    # k = 1: sin(2 pi p), cos(2 pi p)
    np.testing.assert_allclose(f[0, 9:12], [0.0, 0.0, -1.0], atol=1e-7)
    np.testing.assert_allclose(f[0, 12:15], [1.0, -1.0, 0.0], atol=1e-7)
    np.testing.assert_array_equal(f[0, 21:], 0.0)  # zero padding


def test_identity_weight_gives_fp16_input_plus_bias():
    rng = np.random.default_rng(0)
    x = rng.uniform(-3, 3, (64, 16)).astype(np.float32)
    b = rng.uniform(-1, 1, 16).astype(np.float32)
    y = O.linear_fast(x, np.eye(16, dtype=np.float32), b)
    np.testing.assert_array_equal(y, O.f16(x) + b)
    # the fp32 rule keeps x unrounded
    np.testing.assert_array_equal(O.linear_f32(x, np.eye(16, dtype=np.float32), b), x + b)


def test_one_hot_rows_select_columns():
    """W[o] = e_{perm[o]} -> y[:, o] = fp16(x[:, perm[o]]): pins W's [out, in] orientation."""
    rng = np.random.default_rng(1)
    x = rng.uniform(-2, 2, (32, 7)).astype(np.float32)
    perm = np.array([3, 0, 6, 1, 5])
    W = np.zeros((5, 7), np.float32)
    W[np.arange(5), perm] = 1.0
    y = O.linear_fast(x, W, np.zeros(5, np.float32))
    np.testing.assert_array_equal(y, O.f16(x)[:, perm])


def test_zero_weight_gives_bias_and_relu_of_bias():
    x = np.ones((33, 4), np.float32)
    b = np.array([-1.0, 0.5, 2.0], np.float32)
    y = O.mlp_forward(x, [(np.zeros((3, 4), np.float32), b)], ["relu"], ["f16"])
    np.testing.assert_array_equal(y, np.tile(np.maximum(b, 0), (33, 1)))


def test_partial_group_uses_fp32_rule():
    rng = np.random.default_rng(2)
    x = rng.uniform(-1, 1, (45, 8)).astype(np.float32) * 1.37
    W = rng.uniform(-1, 1, (6, 8)).astype(np.float32) * 0.91
    b = np.zeros(6, np.float32)
    y = O.mlp_forward(x, [(W, b)], ["none"], ["f16"])
    np.testing.assert_array_equal(y[:32], O.linear_fast(x[:32], W, b))
    np.testing.assert_array_equal(y[32:], O.linear_f32(x[32:], W, b))
    assert not np.array_equal(y[32:], O.linear_fast(x[32:], W, b))  # the rule is observable


def test_fp16_error_within_reference_statement():
    """linear_fast's fp16 staging costs '~1e-2 max abs error on randn-scale values'
    (src/rdv/domain/nn.py:86-90); the oracle must sit within that of exact fp64."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((256, 64)).astype(np.float32)
    W = (rng.standard_normal((64, 64)) / 8).astype(np.float32)
    exact = x.astype(np.float64) @ W.astype(np.float64).T
    err = np.abs(O.linear_fast(x, W, np.zeros(64, np.float32)) - exact).max()
    assert 1e-5 < err < 1e-2


def test_chain_equals_layer_by_layer():
    rng = np.random.default_rng(4)
    x = rng.uniform(-1, 1, (64, 3)).astype(np.float32)
    layers = [(rng.uniform(-1, 1, (9, 3)).astype(np.float32), rng.uniform(-1, 1, 9).astype(np.float32)),
              (rng.uniform(-1, 1, (4, 9)).astype(np.float32), rng.uniform(-1, 1, 4).astype(np.float32))]
    y = O.mlp_forward(x, layers, ["relu", "none"], ["f16", "f16"])
    h = O.relu(O.linear_fast(x, *layers[0]))
    np.testing.assert_array_equal(y, O.linear_fast(h, *layers[1]))


def test_heads():
    v = np.array([-30.0, -1.0, 0.0, 1.0, 30.0], np.float32)
    np.testing.assert_allclose(O.softplus(v), np.log1p(np.exp(v.astype(np.float64))), rtol=1e-6)
    np.testing.assert_allclose(O.sigmoid(v), 1 / (1 + np.exp(-v.astype(np.float64))), rtol=1e-6)
    d = O.density_rgb(np.array([[0.0, 0.0, 100.0, -100.0]], np.float32))
    np.testing.assert_allclose(d, [[np.log(2.0), 0.5, 1.0, 0.0]], atol=1e-7)


def test_tolerance_helper():
    assert O.within_tolerance([1.0 + 0.0119], [1.0]).all()
    assert not O.within_tolerance([1.0 + 0.0121], [1.0]).all()
    assert O.within_tolerance([0.00199], [0.0]).all()
    assert not O.within_tolerance([0.00201], [0.0]).all()
