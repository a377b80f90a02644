"""Oracle for the linear and ReLU tensor operations — TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

Reference semantics restated (paths relative to /root/reference/src/rdv):
  * LinearTensorOp (domain/nn.py:377-411, shaders/tensors/linear_tensor_op.h:8-51):
    fp32 throughout, acc = bias[o]; acc += x[r][k] * W[o][k] for k ascending
    (:30-46), y[r][o] = acc (:48-50).
  * LinearTensorOpSmall / Simple / Fast / Mine (nn.py:1303-1411, 1204-1300,
    541-605, 1153-1201; shaders/tensors/linear_tensor_op_{small,simple,fast,mine}.h):
    x staged as float16 (e.g. linear_tensor_op_small.h:76-78), W as float16
    (Small/Mine convert at dispatch, Simple and Fast hold fp16 copies made at
    construction, nn.py:472-501), cooperative-matrix products accumulated in
    fp32, fp32 bias (seeded into the accumulator by Small, :99).
  * ReLUTensorOp (nn.py:362-374, shaders/tensors/relu_tensor_op.h:3-22):
    y = max(0.0, x) elementwise.  GLSL leaves max() of a NaN undefined; this
    build defines it as 0.
  * _tile_weight_fp16 (nn.py:472-490): W [out, in] -> [out/16][in/16][16 k][16 n].
The accumulation order of the GPU's fp32 sums is unspecified (matrix-core
products), so parity is to the bound of gemm_error_bound, not bit-exact.
Sums here are formed in float64 and rounded to fp32 once.
"""
from __future__ import annotations

import numpy as np

from . import mlp as M


def linear_op_f32(x, W, b) -> np.ndarray:
    """LinearTensorOp (linear_tensor_op.h:8-51)."""
    return M.linear_f32(np.asarray(x, np.float32), np.asarray(W, np.float32), np.asarray(b, np.float32))


def linear_op_f16(x, W, b) -> np.ndarray:
    """LinearTensorOp{Small,Simple,Fast,Mine}: fp16 x and W, fp32 accumulation and bias."""
    return M.linear_fast(np.asarray(x, np.float32), np.asarray(W, np.float32), np.asarray(b, np.float32))


def relu_op(x) -> np.ndarray:
    """ReLUTensorOp (relu_tensor_op.h:15-19); NaN -> 0."""
    x = np.asarray(x, np.float32)
    return np.where(x > 0, x, np.float32(0)).astype(np.float32)


def gemm_error_bound(x, W, b, f16: bool) -> np.ndarray:
    """Per-element bound on |GPU - oracle| for y = x W^T + b with any fp32
    summation order: gamma_n (sum_k |x_k W_ok| + |b_o|), gamma_n = n u / (1 - n u),
    u = 2^-24, n = in + 2 (the products, the bias and the final rounding)."""
    x = np.asarray(x, np.float64)
    W = np.asarray(W, np.float64)
    if f16:
        x = M.f16(x).astype(np.float64)
        W = M.f16(W).astype(np.float64)
    n = x.shape[1] + 2
    u = 2.0 ** -24
    gamma = n * u / (1 - n * u)
    mag = np.abs(x) @ np.abs(W).T + np.abs(np.asarray(b, np.float64))
    return gamma * mag + 1e-30


def tile_weight_fp16(W) -> np.ndarray:
    """_tile_weight_fp16 (nn.py:472-490): flat fp16, element (o, k) of W at
    ((o // 16) * (in // 16) + k // 16) * 256 + (k % 16) * 16 + o % 16."""
    W = np.asarray(W, np.float32)
    out_features, in_features = W.shape
    t = W.reshape(out_features // 16, 16, in_features // 16, 16).transpose(0, 2, 3, 1)
    return np.ascontiguousarray(t).astype(np.float16).reshape(-1)


def max_subgroups(fixed_bytes, per_subgroup_bytes, divides, budget=49152, cap=32) -> int:
    """_max_subgroups (nn.py:504-519)."""
    spt = 1
    while spt * 2 <= cap and fixed_bytes + spt * 2 * per_subgroup_bytes <= budget and divides(spt * 2):
        spt *= 2
    return spt


# ----------------------------------------------------------- data movement
# Channels-last fp32 images x [H*W, C], row r = h * W + w.  Bit-exact restatements.

def downsample2x(x, H: int, W: int) -> np.ndarray:
    """Downsample2xTensorOp (domain/nn.py:1090-1107, shaders/tensors/downsample2x_tensor_op.h:22-34):
    v = x00 + x01 + x10 + x11 summed left to right in fp32, result v * 0.25."""
    x = np.asarray(x, np.float32).reshape(H, W, -1)
    a, b = x[0::2, 0::2], x[0::2, 1::2]
    c, d = x[1::2, 0::2], x[1::2, 1::2]
    v = ((a + b) + c) + d                      # float32 adds, in the shader's order
    return (v * np.float32(0.25)).reshape((H // 2) * (W // 2), -1)


def upsample2x(x, H: int, W: int) -> np.ndarray:
    """Upsample2xTensorOp (domain/nn.py:1110-1125, shaders/tensors/upsample2x_tensor_op.h:19-27):
    output pixel (oh, ow) copies input pixel (oh // 2, ow // 2)."""
    x = np.asarray(x, np.float32).reshape(H, W, -1)
    return np.repeat(np.repeat(x, 2, axis=0), 2, axis=1).reshape(4 * H * W, -1)


def concat(x1, x2) -> np.ndarray:
    """ConcatTensorOp (domain/nn.py:1128-1150, shaders/tensors/concat_tensor_op.h:19-23):
    columns < C1 from x1, the rest from x2."""
    return np.concatenate([np.asarray(x1, np.float32), np.asarray(x2, np.float32)], axis=1)


# ------------------------------------------------------------ direct conv
def _im2col(x, H: int, W: int, KH: int, KW: int) -> np.ndarray:
    """[H*W, KH*KW*C] patches in the shaders' K order (kh, kw, channel): tap
    (kh, kw) of output pixel (h, w) reads input (h + kh - KH//2, w + kw - KW//2),
    zero outside the image (conv2d_tensor_op.h:27-28, 45-53)."""
    x = np.asarray(x, np.float64).reshape(H, W, -1)
    C = x.shape[2]
    ph, pw = KH // 2, KW // 2
    xp = np.zeros((H + KH - 1, W + KW - 1, C))
    xp[ph:ph + H, pw:pw + W] = x
    cols = [xp[kh:kh + H, kw:kw + W] for kh in range(KH) for kw in range(KW)]
    return np.concatenate(cols, axis=2).reshape(H * W, KH * KW * C)


def conv2d_op_f32(x, w, b, H: int, W: int) -> np.ndarray:
    """Conv2DTensorOp (domain/nn.py:414-470, shaders/tensors/conv2d_tensor_op.h:20-80):
    acc = bias[o]; acc += x[tap pixel][k] * w[kh][kw][k][o] over the valid taps in
    (kh, kw) order and k ascending, fp32.  w is [KH, KW, CIN, COUT]."""
    w = np.asarray(w, np.float32)
    KH, KW, C, K = w.shape
    acc = _im2col(x, H, W, KH, KW) @ w.astype(np.float64).reshape(KH * KW * C, K)
    return (acc + np.asarray(b, np.float64)).astype(np.float32)


def conv2d_op_f16(x, w, b, H: int, W: int) -> np.ndarray:
    """Conv2DTensorOp{Fast,Simple,Simple3x3,Window3x3} (domain/nn.py:608-1000,
    shaders/tensors/conv2d_tensor_op_{fast,simple,simple3x3,window3x3}.h): x and w
    staged as float16 (e.g. conv2d_tensor_op_fast.h:77-86), products summed in
    fp32 over every tap and channel, fp32 bias (seeded by Simple/Simple3x3/
    Window3x3, added after by Fast: the same value up to the fp32 sum order)."""
    w = M.f16(w)
    KH, KW, C, K = w.shape
    acc = _im2col(M.f16(x), H, W, KH, KW) @ w.astype(np.float64).reshape(KH * KW * C, K)
    return (acc + np.asarray(b, np.float64)).astype(np.float32)


def conv2d_error_bound(x, w, b, H: int, W: int, f16: bool) -> np.ndarray:
    """gamma_n (sum |x w| + |b|) per output, n = KH KW CIN + 2: the bound on
    any fp32 summation order of the products (the same argument as
    gemm_error_bound)."""
    w = np.asarray(w, np.float32)
    KH, KW, C, K = w.shape
    xs = M.f16(x) if f16 else np.asarray(x, np.float32)
    ws = M.f16(w) if f16 else w
    mag = np.abs(_im2col(xs, H, W, KH, KW)) @ np.abs(ws.astype(np.float64)).reshape(KH * KW * C, K)
    n = KH * KW * C + 2
    u = 2.0 ** -24
    return (n * u / (1 - n * u)) * (mag + np.abs(np.asarray(b, np.float64)))
