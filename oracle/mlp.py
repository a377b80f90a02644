"""Oracle for fused MLP chains — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference semantics restated (all paths relative to /root/reference/src/rdv):
  * LinearFast on a full 32-row workgroup (shaders/maps/linear_fast.h:61-98):
    input row staged as float16 (:62), weight tile staged as float16 (:82-83),
    16x16x16 cooperative-matrix products accumulated in fp32 (:86-90),
    then `_output[o] = _SH_Y[...] + bias[o]` in fp32 (:97-98).
  * LinearFast on a partial workgroup, and Linear always
    (linear_fast.h:102-108, shaders/maps/linear.h:36-43):
    acc = bias[o]; acc += x[k] * W[o*IN + k] in fp32 (no fp16 rounding).
  * all_thread_sync (shaders/libraries/cooperative_library.h:20-33) is true only
    for a workgroup whose 32 lanes are all live, i.e. every group of 32 rows
    except a partial last one (MapEvaluator workgroup size 32, maths/__init__.py:1591).
  * ReLU (shaders/maps/relu.h:1-5): max(x, 0), elementwise, fp32.
  * Composite (shaders/maps/composite.h:8-12): f(g(x)), row by row.
Sums are formed in float64 and rounded to fp32 once; the hardware's fp32
accumulation order is unspecified (coopMatMulAdd), so parity is to a stated
tolerance, not bit-exact.

Build-defined parts (no reference counterpart): freq_encode, softplus, sigmoid,
density_rgb heads.
"""
from __future__ import annotations

import numpy as np

GROUP = 32  # MapEvaluator workgroup size (maths/__init__.py:1591)


def f16(a) -> np.ndarray:
    """Round to fp16 (RNE) and back to fp32 (GLSL float16_t(), assumed RNE)."""
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def linear_fast(x: np.ndarray, W: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Full-workgroup LinearFast (linear_fast.h:61-98)."""
    acc = f16(x).astype(np.float64) @ f16(W).astype(np.float64).T
    return acc.astype(np.float32) + np.asarray(b, np.float32)


def linear_f32(x: np.ndarray, W: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Linear, and LinearFast's fallback (linear.h:36-43, linear_fast.h:102-108)."""
    acc = np.asarray(b, np.float64) + np.asarray(x, np.float64) @ np.asarray(W, np.float64).T
    return acc.astype(np.float32)


def relu(x: np.ndarray) -> np.ndarray:
    return np.maximum(x, np.float32(0))


def softplus(x: np.ndarray) -> np.ndarray:
    return np.logaddexp(0.0, np.asarray(x, np.float64)).astype(np.float32)


def sigmoid(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float64)
    e = np.exp(-np.abs(x))  # stable for both signs
    return np.where(x >= 0, 1.0 / (1.0 + e), e / (1.0 + e)).astype(np.float32)


def density_rgb(x: np.ndarray) -> np.ndarray:
    out = sigmoid(x)
    out[..., 0] = softplus(x[..., 0])
    return out


ACTS = {
    "none": lambda v: np.asarray(v, np.float32),
    "relu": relu,
    "softplus": softplus,
    "sigmoid": sigmoid,
    "density_rgb": density_rgb,
}


def freq_encode(p: np.ndarray, octaves: int, width: int | None = None) -> np.ndarray:
    """[p, sin(2^k pi p) (D values), cos(2^k pi p) (D values) for k < octaves], zero padded."""
    p64 = np.asarray(p, np.float64)
    feats = [p64]
    for k in range(octaves):
        t = np.pi * (2.0 ** k) * p64
        feats.append(np.sin(t))
        feats.append(np.cos(t))
    out = np.concatenate(feats, axis=-1)
    if width is not None and width > out.shape[-1]:
        pad = np.zeros((*out.shape[:-1], width - out.shape[-1]))
        out = np.concatenate([out, pad], axis=-1)
    return out.astype(np.float32)


def chain(x: np.ndarray, layers, acts, precs, full_group: bool = True) -> np.ndarray:
    """One group of rows through the chain.  layers = [(W, b)], acts = act names,
    precs = 'f16' (LinearFast) or 'f32' (Linear).  full_group=False applies the
    partial-workgroup rule: every layer in fp32."""
    h = np.asarray(x, np.float32)
    for (W, b), a, p in zip(layers, acts, precs):
        h = linear_fast(h, W, b) if (p == "f16" and full_group) else linear_f32(h, W, b)
        h = ACTS[a](h)
    return h


def mlp_forward(x: np.ndarray, layers, acts, precs, encoding: tuple | None = None) -> np.ndarray:
    """Map.__call__ over x[..., IN] (maths/__init__.py:1451-1487): rows in groups
    of 32; a partial last group is evaluated in fp32.  encoding = (octaves, width)
    applies freq_encode first."""
    x = np.asarray(x, np.float32)
    lead = x.shape[:-1]
    rows = x.reshape(-1, x.shape[-1])
    if encoding is not None:
        rows = freq_encode(rows, *encoding)
    n = rows.shape[0]
    n_full = (n // GROUP) * GROUP
    parts = []
    if n_full:
        parts.append(chain(rows[:n_full], layers, acts, precs, True))
    if n > n_full:
        parts.append(chain(rows[n_full:], layers, acts, precs, False))
    out_w = layers[-1][0].shape[0]
    y = np.concatenate(parts, axis=0) if parts else np.zeros((0, out_w), np.float32)
    return y.reshape(*lead, out_w)


def within_tolerance(y, ref, abs_tol=2e-3, rel_tol=1e-2) -> np.ndarray:
    """|y - ref| <= abs + rel * |ref|, elementwise (the fp16 MLP parity bar)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return np.abs(y - ref) <= abs_tol + rel_tol * np.abs(ref)
