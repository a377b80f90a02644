"""Oracle for the Winograd F(2x2,3x3) convolution — TEST INFRASTRUCTURE ONLY
(see oracle/__init__.py).

Reference semantics restated (paths relative to /root/reference/src/rdv):
  * Weight transform (domain/nn.py:522-538): g[ci][co] = w[:, :, ci, co] (a 3x3
    filter), U = G g G^T with G = [[1,0,0],[.5,.5,.5],[.5,-.5,.5],[0,0,1]] in fp32,
    stored as U[p = 4a + b][ci][co] rounded to fp16.
  * Per 2x2 output tile at (oh0, ow0) = (2 * tile_row, 2 * tile_col) and input
    channel ci (shaders/tensors/conv2d_tensor_op_winograd3x3.h:123-137): the 4x4
    input patch d[dr][dc] = x[oh0 - 1 + dr][ow0 - 1 + dc][ci] (zero outside the
    image) is transformed in fp32 by _winograd_fwd (:59-78), V = B^T d B with
    B^T = [[1,0,-1,0],[0,1,1,0],[0,-1,1,0],[0,1,0,-1]], and V[p] rounded to fp16 (:136).
  * M[p][tile][co] = sum over ci of V[p] * U[p] with fp32 accumulation (:142-161).
  * Y = A^T M A with A^T = [[1,1,1,0],[0,1,-1,-1]] (_winograd_inv, :80-93), plus
    the fp32 bias (:169-173); Y[i][j] is output pixel (oh0 + i, ow0 + j).  The
    reference has no activation; the ReLU epilogue of the benchmark configuration
    is applied after the bias.
The transforms are restated in the shader's own fp32 operation order, so U and
V are bit-exact; only M's channel sums (coopMatMulAdd's fp32 accumulation order
is unspecified) are formed in float64 and rounded to fp32 once, so parity is to
a tolerance.

Layouts: x is channels-last [H, W, CIN] (the reference's [H*W, CIN]), w is
[3, 3, CIN, COUT] (the reference's layout), output [H, W, COUT].
"""
from __future__ import annotations

import numpy as np

G = np.array([[1.0, 0.0, 0.0], [0.5, 0.5, 0.5], [0.5, -0.5, 0.5], [0.0, 0.0, 1.0]])
BT = np.array([[1.0, 0.0, -1.0, 0.0], [0.0, 1.0, 1.0, 0.0], [0.0, -1.0, 1.0, 0.0], [0.0, 1.0, 0.0, -1.0]])
AT = np.array([[1.0, 1.0, 1.0, 0.0], [0.0, 1.0, -1.0, -1.0]])


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).astype(np.float32)


def transform_weight(w: np.ndarray, exact: bool = False) -> np.ndarray:
    """w [3, 3, CIN, COUT] -> U [16, CIN, COUT] (nn.py:525-538).

    exact=False follows the reference's fp32 evaluation: T = G g, then
    U = T G^T, each element a left-to-right fp32 sum of 3 products (the
    products are exact: G holds 0, +-0.5 and 1), rounded once to fp16.
    exact=True is the float64 algebra."""
    g = np.asarray(w, np.float64).transpose(2, 3, 0, 1)  # [CIN, COUT, 3(r), 3(s)]
    cin, cout = g.shape[:2]
    if exact:
        U = G @ g @ G.T                                  # [CIN, COUT, 4, 4]
        return U.reshape(cin, cout, 16).transpose(2, 0, 1)
    g = g.astype(np.float32)
    Gf = G.astype(np.float32)
    T = np.empty((cin, cout, 4, 3), np.float32)
    for a in range(4):
        for s_ in range(3):
            acc = Gf[a, 0] * g[:, :, 0, s_]
            acc = acc + Gf[a, 1] * g[:, :, 1, s_]
            T[:, :, a, s_] = acc + Gf[a, 2] * g[:, :, 2, s_]
    U = np.empty((cin, cout, 4, 4), np.float32)
    for a in range(4):
        for b in range(4):
            acc = T[:, :, a, 0] * Gf[b, 0]
            acc = acc + T[:, :, a, 1] * Gf[b, 1]
            U[:, :, a, b] = acc + T[:, :, a, 2] * Gf[b, 2]
    return f16(U.reshape(cin, cout, 16).transpose(2, 0, 1))


def input_patches(x: np.ndarray) -> np.ndarray:
    """x [H, W, CIN] -> d [TH, TW, CIN, 4, 4], the zero-padded 4x4 patches
    (.h:123-134: d[dr][dc] = x[oh0 - 1 + dr][ow0 - 1 + dc], 0 outside)."""
    H, W, C = x.shape
    xp = np.zeros((H + 2, W + 2, C), dtype=x.dtype)
    xp[1:H + 1, 1:W + 1] = x
    TH, TW = H // 2, W // 2
    d = np.empty((TH, TW, C, 4, 4), dtype=x.dtype)
    for dr in range(4):
        for dc in range(4):
            d[:, :, :, dr, dc] = xp[dr:dr + 2 * TH:2, dc:dc + 2 * TW:2, :]
    return d


def winograd_fwd_f32(d: np.ndarray) -> np.ndarray:
    """V = B^T d B over the trailing [4, 4] axes in fp32, in the operation
    order of _winograd_fwd (.h:59-78): columns first (m = B^T d), then rows."""
    d = np.asarray(d, np.float32)
    m = np.empty_like(d)
    d0, d1, d2, d3 = d[..., 0, :], d[..., 1, :], d[..., 2, :], d[..., 3, :]
    m[..., 0, :] = d0 - d2
    m[..., 1, :] = d1 + d2
    m[..., 2, :] = d2 - d1
    m[..., 3, :] = d1 - d3
    V = np.empty_like(d)
    m0, m1, m2, m3 = m[..., 0], m[..., 1], m[..., 2], m[..., 3]
    V[..., 0] = m0 - m2
    V[..., 1] = m1 + m2
    V[..., 2] = m2 - m1
    V[..., 3] = m1 - m3
    return V


def winograd_inv_f32(M: np.ndarray) -> np.ndarray:
    """Y = A^T M A over the trailing [4, 4] axes in fp32, in the operation
    order of _winograd_inv (.h:80-93).  Returns [..., 2, 2]."""
    M = np.asarray(M, np.float32)
    t0 = M[..., 0, :] + M[..., 1, :] + M[..., 2, :]   # [..., 4] over columns
    t1 = M[..., 1, :] - M[..., 2, :] - M[..., 3, :]
    Y = np.empty(M.shape[:-2] + (2, 2), np.float32)
    for i, t in enumerate((t0, t1)):
        Y[..., i, 0] = t[..., 0] + t[..., 1] + t[..., 2]
        Y[..., i, 1] = t[..., 1] - t[..., 2] - t[..., 3]
    return Y


def winograd_conv(x: np.ndarray, w: np.ndarray, b=None, relu: bool = False, exact: bool = False) -> np.ndarray:
    """The reference Winograd path on channels-last x [H, W, CIN].

    exact=False mirrors the reference's arithmetic: U and V rounded to fp16
    after fp32 transforms in the shader's operation order, M accumulated (here
    in float64, rounded once to fp32: the matrix-core summation order is
    unspecified), inverse transform and bias add in fp32.  exact=True is the
    float64 algebra, which equals direct_conv to ~1e-12."""
    H, W, C = x.shape
    assert H % 2 == 0 and W % 2 == 0
    U = transform_weight(w, exact=exact).astype(np.float64)             # [16, C, K]
    if exact:
        d = input_patches(np.asarray(x, np.float64))
        V = BT @ d @ BT.T                                                # [TH, TW, C, 4, 4]
    else:
        d = input_patches(np.asarray(x, np.float32))
        V = f16(winograd_fwd_f32(d)).astype(np.float64)
    V = V.reshape(*V.shape[:3], 16)                                      # [TH, TW, C, 16]
    M = np.einsum("hwcp,pck->hwkp", V, U, optimize=True)                 # [TH, TW, K, 16]
    M = M.reshape(*M.shape[:3], 4, 4)
    if exact:
        Y = AT @ M @ AT.T                                                # [TH, TW, K, 2, 2]
    else:
        Y = winograd_inv_f32(M.astype(np.float32))
    K = Y.shape[2]
    out = Y.transpose(0, 3, 1, 4, 2).reshape(H, W, K)
    if b is not None:
        out = out + np.asarray(b, out.dtype)
    if relu:
        out = np.maximum(out, 0)
    return out


def direct_conv(x: np.ndarray, w: np.ndarray, b=None, relu: bool = False) -> np.ndarray:
    """'same'-padded stride-1 3x3 cross-correlation in float64:
    out[oh][ow][co] = sum x[oh-1+r][ow-1+s][ci] * w[r][s][ci][co]."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    H, W, C = x.shape
    xp = np.zeros((H + 2, W + 2, C))
    xp[1:H + 1, 1:W + 1] = x
    out = np.zeros((H, W, w.shape[3]))
    for r in range(3):
        for s in range(3):
            out += xp[r:r + H, s:s + W, :] @ w[r, s]
    if b is not None:
        out = out + np.asarray(b, np.float64)
    if relu:
        out = np.maximum(out, 0.0)
    return out
