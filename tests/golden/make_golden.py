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
    print("wrote", len(cases) + 1, "fixtures to", HERE)


if __name__ == "__main__":
    main()
