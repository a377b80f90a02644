"""Oracle for the MLP training step (forward, MSE, backward) — TEST
INFRASTRUCTURE ONLY (see oracle/__init__.py).

Build-defined (the reference has no backward pass for this path).  The forward
is the LinearFast chain of oracle.mlp (fp16 layer inputs and weights, fp32
accumulation, fp32 bias, ReLU hidden layers, linear head).  The loss is the mean
over n x out of (y - t)^2.  The gradients are those of that forward function
with every fp16 rounding treated as the identity (the straight-through
convention of autograd through a cast), computed in float64:
    dz_L = 2 (y - t) / (n out);  dW_l = dz_{l+1}^T h_l;  db_l = sum_p dz_{l+1}
    dz_l = (dz_{l+1} W_l) * [h_l > 0]
where h_l is layer l's fp16 input.
"""
from __future__ import annotations

import numpy as np

from . import mlp as M


def forward_states(x, layers):
    """fp16-rounded layer inputs h_0..h_{L-1} (float64) and the fp32 output y."""
    hs = []
    h = M.f16(np.asarray(x, np.float32)).astype(np.float64)
    for i, (W, b) in enumerate(layers):
        hs.append(h)
        y = M.linear_fast(h.astype(np.float32), W, b)
        if i + 1 < len(layers):
            h = M.f16(np.maximum(y, 0.0)).astype(np.float64)
    return hs, y.astype(np.float64)


def mse_grads(x, layers, target):
    """(loss, [(dW_l, db_l)]) of the chain on x [n, in] against target [n, out]."""
    hs, y = forward_states(x, layers)
    t = np.asarray(target, np.float64)
    n, out = y.shape
    loss = np.mean((y - t) ** 2)
    dz = 2.0 * (y - t) / (n * out)
    grads = [None] * len(layers)
    for l in range(len(layers) - 1, -1, -1):
        W = M.f16(np.asarray(layers[l][0], np.float32)).astype(np.float64)
        grads[l] = (dz.T @ hs[l], dz.sum(axis=0))
        if l > 0:
            dz = (dz @ W) * (hs[l] > 0)
    return loss, grads
