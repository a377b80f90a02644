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
