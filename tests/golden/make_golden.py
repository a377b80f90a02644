"""Writes tests/golden/*.npz: small known-answer vectors computed by scalar
pure-Python loops written straight from the reference's shader text.

The reference itself cannot run here (it needs the `vulky` Vulkan binding and a
Vulkan device; neither exists in this image), and it ships no fixtures of its
own for this path.  These vectors therefore pin the numpy oracle against an
independent scalar restatement: per-element loops, Python floats (binary64),
fp16 rounding via struct's IEEE half format (round-half-even) and fp32 rounding
via struct's IEEE single format.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def r16(v: float) -> float:
    return struct.unpack("<e", struct.pack("<e", v))[0]


def r32(v: float) -> float:
    return struct.unpack("<f", struct.pack("<f", v))[0]


def lcg(seed: int):
    """Deterministic pseudo-random floats in [-1, 1) (no numpy RNG dependence)."""
    s = seed & 0xFFFFFFFF
    while True:
        s = (1664525 * s + 1013904223) & 0xFFFFFFFF
        yield (s / 2 ** 32) * 2.0 - 1.0


def take(g, n):
    return [next(g) for _ in range(n)]


def linear_fast_row(x, W, b):
    """linear_fast.h:61-98 for one row: fp16 input and weight, fp32 sum, + fp32 bias."""
    out = []
    for o in range(len(W)):
        s = 0.0
        for k in range(len(x)):
            s += r16(x[k]) * r16(W[o][k])  # each product and the running sum are exact in binary64 here
        out.append(r32(r32(s) + b[o]))
    return out


def linear_f32_row(x, W, b):
    """linear.h:36-43: acc = b; acc += x[k] * W[o][k], sum formed exactly then rounded to fp32."""
    out = []
    for o in range(len(W)):
        s = b[o]
        for k in range(len(x)):
            s += x[k] * W[o][k]
        out.append(r32(s))
    return out


def chain_rows(X, layers, acts, precs):
    Y = []
    n = len(X)
    n_full = (n // 32) * 32
    for i, x in enumerate(X):
        full = i < n_full
        h = list(x)
        for (W, b), a, p in zip(layers, acts, precs):
            h = linear_fast_row(h, W, b) if (p == "f16" and full) else linear_f32_row(h, W, b)
            if a == "relu":
                h = [max(v, 0.0) for v in h]
        Y.append(h)
    return Y


def make_chain_case(seed, n, dims, acts, precs):
    g = lcg(seed)
    X = [[r32(v) for v in take(g, dims[0])] for _ in range(n)]
    layers = []
    for i in range(len(dims) - 1):
        W = [[r32(v * math.sqrt(6.0 / dims[i])) for v in take(g, dims[i])] for _ in range(dims[i + 1])]
        b = [r32(0.1 * v) for v in take(g, dims[i + 1])]
        layers.append((W, b))
    Y = chain_rows(X, layers, acts, precs)
    arrays = {"x": np.array(X, np.float32), "y": np.array(Y, np.float32),
              "dims": np.array(dims, np.int32), "acts": np.array(acts), "precs": np.array(precs)}
    for i, (W, b) in enumerate(layers):
        arrays[f"W{i}"] = np.array(W, np.float32)
        arrays[f"b{i}"] = np.array(b, np.float32)
    return arrays


def make_freq_case():
    """gamma(p) = [p, sin(2^k pi p), cos(2^k pi p)] for p on a grid including exact points."""
    ps = [0.0, 0.5, -0.5, 0.25, 1.0, -1.0, 0.125, 1.0 / 3.0, -0.7, 0.9]
    P = [[r32(ps[i]), r32(ps[(i + 3) % len(ps)]), r32(ps[(i + 7) % len(ps)])] for i in range(len(ps))]
    L = 6
    F = []
    for p in P:
        f = list(p)
        for k in range(L):
            f += [math.sin(math.pi * (2 ** k) * v) for v in p]
            f += [math.cos(math.pi * (2 ** k) * v) for v in p]
        F.append(f)
    return {"p": np.array(P, np.float32), "features": np.array(F, np.float64), "octaves": np.array(L)}


WG_G = [[1.0, 0.0, 0.0], [0.5, 0.5, 0.5], [0.5, -0.5, 0.5], [0.0, 0.0, 1.0]]


def winograd_u_scalar(w, cin, cout):
    """_winograd_transform_weight (nn.py:525-538) per element: T = G g, U = T G^T,
    each a left-to-right fp32 sum of three products, then fp16.  w[r][s][ci][co]."""
    U = [[[0.0] * cout for _ in range(cin)] for _ in range(16)]
    for ci in range(cin):
        for co in range(cout):
            g = [[w[r][s][ci][co] for s in range(3)] for r in range(3)]
            T = [[r32(r32(r32(WG_G[a][0] * g[0][s]) + r32(WG_G[a][1] * g[1][s])) + r32(WG_G[a][2] * g[2][s]))
                  for s in range(3)] for a in range(4)]
            for a in range(4):
                for b in range(4):
                    v = r32(r32(r32(T[a][0] * WG_G[b][0]) + r32(T[a][1] * WG_G[b][1])) + r32(T[a][2] * WG_G[b][2]))
                    U[4 * a + b][ci][co] = r16(v)
    return U


def winograd_conv_scalar(x, w, bias, H, W, cin, cout):
    """conv2d_tensor_op_winograd3x3.h:95-178 for every tile, written as the
    shader's per-lane loops: d from x (0 outside), _winograd_fwd in fp32, V[p]
    to fp16, M[p] = sum over ci of V*U (exact in binary64, one fp32 rounding),
    _winograd_inv in fp32, + bias.  x[(h * W + w) * cin + c], result likewise."""
    U = winograd_u_scalar(w, cin, cout)
    y = [0.0] * (H * W * cout)
    for tr in range(H // 2):
        for tc in range(W // 2):
            oh0, ow0 = 2 * tr, 2 * tc
            Vall = []
            for c in range(cin):
                d = [0.0] * 16
                for dr in range(4):
                    for dc in range(4):
                        gh, gw = oh0 - 1 + dr, ow0 - 1 + dc
                        d[dr * 4 + dc] = x[(gh * W + gw) * cin + c] if 0 <= gh < H and 0 <= gw < W else 0.0
                m = [0.0] * 16
                for j in range(4):
                    d0, d1, d2, d3 = d[j], d[4 + j], d[8 + j], d[12 + j]
                    m[j], m[4 + j], m[8 + j], m[12 + j] = r32(d0 - d2), r32(d1 + d2), r32(d2 - d1), r32(d1 - d3)
                V = [0.0] * 16
                for i in range(4):
                    m0, m1, m2, m3 = m[4 * i], m[4 * i + 1], m[4 * i + 2], m[4 * i + 3]
                    V[4 * i], V[4 * i + 1], V[4 * i + 2], V[4 * i + 3] = (r32(m0 - m2), r32(m1 + m2), r32(m2 - m1),
                                                                          r32(m1 - m3))
                Vall.append([r16(v) for v in V])
            for co in range(cout):
                M = [r32(sum(Vall[c][p] * U[p][c][co] for c in range(cin))) for p in range(16)]
                t = [0.0] * 8
                for j in range(4):
                    t[j] = r32(r32(M[j] + M[4 + j]) + M[8 + j])
                    t[4 + j] = r32(r32(M[4 + j] - M[8 + j]) - M[12 + j])
                Y = [0.0] * 4
                for i in range(2):
                    Y[2 * i] = r32(r32(t[4 * i] + t[4 * i + 1]) + t[4 * i + 2])
                    Y[2 * i + 1] = r32(r32(t[4 * i + 1] - t[4 * i + 2]) - t[4 * i + 3])
                for k, (dh, dw) in enumerate(((0, 0), (0, 1), (1, 0), (1, 1))):
                    y[((oh0 + dh) * W + ow0 + dw) * cout + co] = r32(Y[k] + bias[co])
    return U, y


def make_winograd_case(seed, H, W, cin, cout):
    g = lcg(seed)
    x = [r32(v) for v in take(g, H * W * cin)]
    wf = [r32(0.3 * v) for v in take(g, 9 * cin * cout)]
    w = [[[[wf[((r * 3 + s) * cin + ci) * cout + co] for co in range(cout)] for ci in range(cin)] for s in range(3)]
         for r in range(3)]
    bias = [r32(0.1 * v) for v in take(g, cout)]
    U, y = winograd_conv_scalar(x, w, bias, H, W, cin, cout)
    return {
        "x": np.array(x, np.float32).reshape(H, W, cin),
        "w": np.array(wf, np.float32).reshape(3, 3, cin, cout),
        "b": np.array(bias, np.float32),
        "U": np.array(U, np.float32),
        "y": np.array(y, np.float32).reshape(H, W, cout),
    }


def main():
    cases = {
        # 40 rows: one full group of 32 (fp16 path) + a partial group of 8 (fp32 rule)
        "chain_f16_3_5_2": make_chain_case(11, 40, [3, 5, 2], ["relu", "none"], ["f16", "f16"]),
        "chain_f16_16_24_8_4": make_chain_case(12, 70, [16, 24, 8, 4], ["relu", "relu", "none"],
                                               ["f16", "f16", "f16"]),
        "chain_f32_4_6_3": make_chain_case(13, 10, [4, 6, 3], ["relu", "none"], ["f32", "f32"]),
        "chain_mixed_5_7_3": make_chain_case(14, 35, [5, 7, 3], ["relu", "none"], ["f32", "f16"]),
    }
    for name, arrays in cases.items():
        np.savez(os.path.join(HERE, f"{name}.npz"), **arrays)
    np.savez(os.path.join(HERE, "freq_encoding.npz"), **make_freq_case())
    wcases = {
        "winograd_6x8_5_16": make_winograd_case(21, 6, 8, 5, 16),
        "winograd_4x4_16_32": make_winograd_case(22, 4, 4, 16, 32),
    }
    for name, arrays in wcases.items():
        np.savez(os.path.join(HERE, f"{name}.npz"), **arrays)
    print("wrote", len(cases) + 1 + len(wcases), "fixtures to", HERE)


if __name__ == "__main__":
    main()
