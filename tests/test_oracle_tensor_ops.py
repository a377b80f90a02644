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


# ----------------------------------------------------------- data movement

def _brute_downsample(x, H, W):
    """downsample2x_tensor_op.h:22-34 literally, one output element at a time."""
    C = x.shape[1]
    y = np.zeros(((H // 2) * (W // 2), C), np.float32)
    for oh in range(H // 2):
        for ow in range(W // 2):
            for c in range(C):
                v = np.float32(x[(2 * oh) * W + 2 * ow, c])
                v = np.float32(v + x[(2 * oh) * W + 2 * ow + 1, c])
                v = np.float32(v + x[(2 * oh + 1) * W + 2 * ow, c])
                v = np.float32(v + x[(2 * oh + 1) * W + 2 * ow + 1, c])
                y[oh * (W // 2) + ow, c] = np.float32(v * np.float32(0.25))
    return y


def test_downsample_oracle_brute_force_and_avg_pool():
    H, W, C = 6, 10, 8
    x = rng.standard_normal((H * W, C)).astype(np.float32)
    np.testing.assert_array_equal(T.downsample2x(x, H, W), _brute_downsample(x, H, W))
    # integer-valued input: every sum is exact, so any summation order equals torch's average pool
    xi = rng.integers(-50, 50, (H * W, C)).astype(np.float32)
    pool = torch.nn.functional.avg_pool2d(torch.from_numpy(xi).reshape(1, H, W, C).permute(0, 3, 1, 2), 2)
    np.testing.assert_array_equal(T.downsample2x(xi, H, W), pool.permute(0, 2, 3, 1).reshape(-1, C).numpy())


def test_downsample_oracle_sum_order_matters():
    """Values whose fp32 sum depends on the order: the oracle must follow the
    shader's left-to-right order, and a reordered sum differs."""
    x = np.zeros((4, 1), np.float32)
    x[:, 0] = [1e8, 1.0, -1e8, 1.0]  # 2x2 image, taps x00, x01, x10, x11
    got = T.downsample2x(x, 2, 2)[0, 0]
    assert got == np.float32((((np.float32(1e8) + np.float32(1)) + np.float32(-1e8)) + np.float32(1)) * 0.25)
    reordered = np.float32(((np.float32(1e8) + np.float32(-1e8)) + np.float32(1) + np.float32(1)) * 0.25)
    assert got != reordered


def test_upsample_oracle_nearest():
    H, W, C = 3, 5, 8
    x = rng.standard_normal((H * W, C)).astype(np.float32)
    up = T.upsample2x(x, H, W)
    ref = torch.nn.functional.interpolate(torch.from_numpy(x).reshape(1, H, W, C).permute(0, 3, 1, 2),
                                          scale_factor=2, mode="nearest")
    np.testing.assert_array_equal(up, ref.permute(0, 2, 3, 1).reshape(-1, C).numpy())
    for oh in range(2 * H):       # output (oh, ow) copies input (oh // 2, ow // 2)
        for ow in range(2 * W):
            np.testing.assert_array_equal(up[oh * 2 * W + ow], x[(oh // 2) * W + ow // 2])


def test_concat_oracle_columns():
    a = rng.standard_normal((12, 8)).astype(np.float32)
    b = rng.standard_normal((12, 16)).astype(np.float32)
    y = T.concat(a, b)
    np.testing.assert_array_equal(y[:, :8], a)
    np.testing.assert_array_equal(y[:, 8:], b)


# ------------------------------------------------------------ direct conv

def _brute_conv_f32(x, w, b, H, W):
    """conv2d_tensor_op.h:42-73 literally: acc = bias; per tap (kh, kw) in order,
    skip taps outside the image, acc += x * w for k ascending, fp32."""
    KH, KW, C, K = w.shape
    y = np.zeros((H * W, K), np.float32)
    for h in range(H):
        for ww in range(W):
            for o in range(K):
                acc = np.float32(b[o])
                for kh in range(KH):
                    for kw in range(KW):
                        ih, iw = h + kh - KH // 2, ww + kw - KW // 2
                        if not (0 <= ih < H and 0 <= iw < W):
                            continue
                        for k in range(C):
                            acc = np.float32(acc + np.float32(x[ih * W + iw, k] * w[kh, kw, k, o]))
                y[h * W + ww, o] = acc
    return y


@pytest.mark.parametrize("KH,KW", [(3, 3), (1, 1), (2, 2), (3, 5)])
def test_conv_oracle_brute_force(KH, KW):
    H, W, C, K = 5, 6, 8, 8
    x = rng.standard_normal((H * W, C)).astype(np.float32)
    w = (rng.standard_normal((KH, KW, C, K)) * 0.3).astype(np.float32)
    b = rng.standard_normal(K).astype(np.float32)
    got = T.conv2d_op_f32(x, w, b, H, W)
    ref = _brute_conv_f32(x, w, b, H, W)
    assert (np.abs(got - ref) <= 2 * T.conv2d_error_bound(x, w, b, H, W, False) + 1e-30).all()


@pytest.mark.parametrize("KH,KW", [(3, 3), (5, 5), (2, 4), (1, 3)])
def test_conv_oracle_matches_torch(KH, KW):
    """torch's correlation in float64 with the reference's padding (KH//2 rows
    above, the rest below; KW//2 columns to the left)."""
    H, W, C, K = 9, 7, 16, 24
    x = rng.standard_normal((H * W, C)).astype(np.float32)
    w = rng.standard_normal((KH, KW, C, K)).astype(np.float32)
    b = rng.standard_normal(K).astype(np.float32)
    xt = torch.from_numpy(x.astype(np.float64)).reshape(1, H, W, C).permute(0, 3, 1, 2)
    xt = torch.nn.functional.pad(xt, (KW // 2, KW - 1 - KW // 2, KH // 2, KH - 1 - KH // 2))
    wt = torch.from_numpy(w.astype(np.float64)).permute(3, 2, 0, 1)
    ref = torch.nn.functional.conv2d(xt, wt, torch.from_numpy(b.astype(np.float64)))
    ref = ref.permute(0, 2, 3, 1).reshape(H * W, K).numpy()
    np.testing.assert_allclose(T.conv2d_op_f32(x, w, b, H, W), ref, rtol=1e-5, atol=1e-5)
    # fp16 variant: torch on the fp16-rounded operands
    xh = torch.from_numpy(M.f16(x).astype(np.float64)).reshape(1, H, W, C).permute(0, 3, 1, 2)
    xh = torch.nn.functional.pad(xh, (KW // 2, KW - 1 - KW // 2, KH // 2, KH - 1 - KH // 2))
    wh = torch.from_numpy(M.f16(w).astype(np.float64)).permute(3, 2, 0, 1)
    refh = torch.nn.functional.conv2d(xh, wh, torch.from_numpy(b.astype(np.float64)))
    np.testing.assert_allclose(T.conv2d_op_f16(x, w, b, H, W), refh.permute(0, 2, 3, 1).reshape(H * W, K).numpy(),
                               rtol=1e-5, atol=1e-5)


def test_conv_oracle_catches_planted_mistakes():
    """A spatially flipped kernel or swapped kh / kw (a plausible transposition)
    gives a different answer; the one-hot kernel picks a shifted pixel."""
    H, W, C, K = 6, 6, 8, 8
    x = rng.standard_normal((H * W, C)).astype(np.float32)
    w = rng.standard_normal((3, 3, C, K)).astype(np.float32)
    b = np.zeros(K, np.float32)
    y = T.conv2d_op_f32(x, w, b, H, W)
    assert not np.allclose(y, T.conv2d_op_f32(x, w[::-1, ::-1].copy(), b, H, W), atol=1e-3)
    assert not np.allclose(y, T.conv2d_op_f32(x, w.transpose(1, 0, 2, 3).copy(), b, H, W), atol=1e-3)
    # one-hot tap (kh, kw) = (0, 2), channel 3 -> output channel 5 reads x at (h - 1, w + 1)
    e = np.zeros((3, 3, C, K), np.float32)
    e[0, 2, 3, 5] = 1.0
    ys = T.conv2d_op_f32(x, e, b, H, W).reshape(H, W, K)[..., 5]
    xs = x.reshape(H, W, C)[..., 3]
    want = np.zeros((H, W), np.float32)
    want[1:, :-1] = xs[:-1, 1:]
    np.testing.assert_array_equal(ys, want)
