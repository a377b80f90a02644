"""Pins oracle/tensor_ops.py (CPU only): a brute-force loop in the reference's
own accumulation order, an independent library routine (torch.nn.functional
.linear in float64), closed forms that fix the orientation of W, the bias and
the fp16 rounding, and planted mistakes that those checks must catch."""
import numpy as np
import pytest
import torch

from oracle import mlp as M
from oracle import tensor_ops as T

rng = np.random.default_rng(7)


def _case(batch, inf, outf, scale=1.0):
    x = (rng.standard_normal((batch, inf)) * scale).astype(np.float32)
    W = (rng.standard_normal((outf, inf)) / np.sqrt(inf)).astype(np.float32)
    b = rng.standard_normal(outf).astype(np.float32)
    return x, W, b


def _brute_f32(x, W, b):
    """linear_tensor_op.h:30-50 literally: acc = bias; acc += x * w, fp32, k ascending."""
    y = np.zeros((x.shape[0], W.shape[0]), np.float32)
    for r in range(x.shape[0]):
        for o in range(W.shape[0]):
            acc = np.float32(b[o])
            for k in range(x.shape[1]):
                acc = np.float32(acc + np.float32(x[r, k] * W[o, k]))
            y[r, o] = acc
    return y


def _within_bound(got, ref, bound):
    return bool(np.all(np.abs(got.astype(np.float64) - ref.astype(np.float64)) <= bound))


@pytest.mark.parametrize("shape", [(4, 8, 8), (8, 24, 16), (12, 40, 8)])
def test_f32_matches_sequential_brute_force(shape):
    x, W, b = _case(*shape)
    got = T.linear_op_f32(x, W, b)
    ref = _brute_f32(x, W, b)
    assert _within_bound(got, ref, 2 * T.gemm_error_bound(x, W, b, f16=False))


def test_f32_bound_detects_a_dropped_term():
    x, W, b = _case(8, 24, 16)
    ref = _brute_f32(x, W, b)
    bad = T.linear_op_f32(x[:, :-1], W[:, :-1], b)  # the last k is dropped
    assert not _within_bound(bad, ref, 2 * T.gemm_error_bound(x, W, b, f16=False))


@pytest.mark.parametrize("f16", [False, True])
def test_matches_torch_linear(f16):
    x, W, b = _case(64, 48, 32, scale=3.0)
    fn = T.linear_op_f16 if f16 else T.linear_op_f32
    got = fn(x, W, b)
    xt, Wt, bt = torch.from_numpy(x), torch.from_numpy(W), torch.from_numpy(b)
    if f16:  # fp16 operands, fp32 product sum, fp32 bias add
        ref = torch.nn.functional.linear(xt.half().double(), Wt.half().double()).float() + bt
    else:  # one rounding of the exact sum
        ref = torch.nn.functional.linear(xt.double(), Wt.double(), bt.double()).float()
    np.testing.assert_allclose(got, ref.numpy(), rtol=2e-7, atol=1e-6)


@pytest.mark.parametrize("f16", [False, True])
def test_one_hot_rows_select_weight_columns(f16):
    # x[r] = e_k gives y[r] = W[:, k] + b: fixes which index of W is the input one
    inf, outf = 24, 40
    _, W, b = _case(1, inf, outf)
    x = np.eye(inf, dtype=np.float32)
    fn = T.linear_op_f16 if f16 else T.linear_op_f32
    Wr = M.f16(W) if f16 else W
    np.testing.assert_array_equal(fn(x, W, b), (Wr.T + b).astype(np.float32))


def test_transposed_weight_is_caught():
    inf, outf = 24, 24
    _, W, b = _case(1, inf, outf)
    x = np.eye(inf, dtype=np.float32)
    bad = T.linear_op_f32(x, W.T.copy(), b)
    assert not np.array_equal(bad, (W.T + b).astype(np.float32))


def test_identity_weight_and_fp16_rounding():
    # W = I: fp32 path returns x + b, fp16 path returns f16(x) + b
    n = 16
    x = np.full((4, n), 1.0 + 2.0 ** -12, np.float32)  # not representable in fp16 (rounds to 1)
    W = np.eye(n, dtype=np.float32)
    b = np.zeros(n, np.float32)
    np.testing.assert_array_equal(T.linear_op_f32(x, W, b), x)
    np.testing.assert_array_equal(T.linear_op_f16(x, W, b), np.ones_like(x))
    # a path that skipped the fp16 rounding would return x here
    assert not np.array_equal(T.linear_op_f32(x, W, b), T.linear_op_f16(x, W, b))


def test_bias_enters_once():
    x = np.zeros((4, 16), np.float32)
    _, W, b = _case(1, 16, 8)
    np.testing.assert_array_equal(T.linear_op_f32(x, W, b), np.broadcast_to(b, (4, 8)))
    np.testing.assert_array_equal(T.linear_op_f16(x, W, b), np.broadcast_to(b, (4, 8)))


def test_relu_special_values():
    x = np.array([[np.nan, -np.inf, np.inf, -0.0, 0.0, -1.5, 2.5, 1e-45]], np.float32)
    y = T.relu_op(x)
    np.testing.assert_array_equal(y, np.array([[0, 0, np.inf, 0, 0, 0, 2.5, 1e-45]], np.float32))
    assert not np.isnan(y).any()


def test_tile_weight_index_formula():
    # W[o, k] = o * in + k encodes the position; every value is exact in fp16 (< 2048)
    outf, inf = 32, 48
    W = (np.arange(outf)[:, None] * inf + np.arange(inf)[None, :]).astype(np.float32)
    flat = T.tile_weight_fp16(W)
    assert flat.dtype == np.float16 and flat.size == outf * inf
    for idx in range(flat.size):
        blk, rem = divmod(idx, 256)
        nt, kt = divmod(blk, inf // 16)
        k_local, n_local = divmod(rem, 16)
        o, k = nt * 16 + n_local, kt * 16 + k_local
        assert flat[idx] == W[o, k], (idx, o, k)


def test_tile_weight_planted_swap_is_caught():
    outf, inf = 32, 32
    W = (np.arange(outf)[:, None] * inf + np.arange(inf)[None, :]).astype(np.float32)
    # k_local and n_local swapped (the [N, K] tile order the reference avoids, nn.py:484-487)
    bad = W.reshape(2, 16, 2, 16).transpose(0, 2, 1, 3).astype(np.float16).reshape(-1)
    assert not np.array_equal(bad, T.tile_weight_fp16(W))


def test_max_subgroups_closed_forms():
    # LinearTensorOpSmall 128 -> 128 at batch % 64 == 0: 32768 + 2 * 8192 = 49152 fits, 4 does not
    assert T.max_subgroups(128 * 128 * 2, 32 * 128 * 2, lambda s: 4096 % (32 * s) == 0) == 2
    # ... and batch 96 (not a multiple of 64) keeps 1
    assert T.max_subgroups(128 * 128 * 2, 32 * 128 * 2, lambda s: 96 % (32 * s) == 0) == 1
    # LinearTensorOpSimple in = 128: 8192 + 8 * 4096 = 40960 fits, 16 does not
    assert T.max_subgroups(32 * 128 * 2, 16 * 128 * 2, lambda s: 128 % (16 * s) == 0) == 8
    # ... out = 48 only allows s = 1 (48 % 32 != 0)
    assert T.max_subgroups(32 * 128 * 2, 16 * 128 * 2, lambda s: 48 % (16 * s) == 0) == 1
