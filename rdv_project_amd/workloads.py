"""Seeded synthetic inputs for the benchmark configurations.

All tensors are drawn on the CPU from torch.Generator(seed) and returned on the
CPU; callers move them to the GPU.  Weights are Kaiming-uniform,
U(-sqrt(6/fan_in), +sqrt(6/fan_in)) with fan_in the unpadded input width, drawn
per layer in layer order from one generator, rounded to fp16 and returned as
fp32 (exact).  Biases are zero.  Padded weight columns are zero.

  C1  65,536 pts, x ~ U[-1,1]^3 (seed 0), 3->64->64->64->64->4, ReLU, W seed 1
  C2  2^20 pts, x ~ U[-1,1]^3 (seed 0), FREQ(6 octaves) 39 -> pad 48 ->64->64->64->4, W seed 1
  C3  Winograd 1x64x256x256 fp16 in [0,1] (seed 3), w ~ N(0, sqrt(2/576)) (seed 4), bias 0, ReLU
  C4  512x512 rays x 128 samples, MLP 3->64->64->64->4 (seed 2), density+RGB head
  C5  4,194,304 pts, x ~ N(0,1) fp16 (seed 5), target N(0,1) (seed 6), 32->128x8->16, W seed 7
"""
from __future__ import annotations

import math

import torch


def gen(seed: int) -> torch.Generator:
    g = torch.Generator(device="cpu")
    g.manual_seed(seed)
    return g


def kaiming_uniform_f16(shapes, seed: int, fan_ins=None, padded_in=None):
    """[(W fp32 with fp16 values, b zeros)] for layer shapes [(out, in)]."""
    g = gen(seed)
    layers = []
    for i, (o, k) in enumerate(shapes):
        fan = fan_ins[i] if fan_ins else k
        bound = math.sqrt(6.0 / fan)
        w = (torch.rand(o, fan, generator=g) * 2.0 - 1.0) * bound
        w = w.half().float()
        width = padded_in[i] if padded_in and padded_in[i] else k
        if width > fan:
            w = torch.cat([w, torch.zeros(o, width - fan)], dim=1)
        layers.append((w.contiguous(), torch.zeros(o)))
    return layers


def c1(n: int = 65536):
    x = torch.rand(n, 3, generator=gen(0)) * 2.0 - 1.0
    layers = kaiming_uniform_f16([(64, 3), (64, 64), (64, 64), (64, 64), (4, 64)], seed=1)
    return x, layers


C2_OCTAVES = 6
C2_ENC = 3 * (1 + 2 * C2_OCTAVES)  # 39
C2_PAD = 48


def c2(n: int = 1 << 20):
    x = torch.rand(n, 3, generator=gen(0)) * 2.0 - 1.0
    layers = kaiming_uniform_f16([(64, C2_PAD), (64, 64), (64, 64), (4, 64)], seed=1,
                                 fan_ins=[C2_ENC, 64, 64, 64], padded_in=[C2_PAD, 0, 0, 0])
    return x, layers


def c4_mlp():
    return kaiming_uniform_f16([(64, 3), (64, 64), (64, 64), (4, 64)], seed=2)


C4_WIDTH = 512
C4_HEIGHT = 512
C4_SAMPLES = 128


def c4_pose():
    """[1, 9] = origin | target | up (rdv Cameras pose layout, rendering.py:24-42)."""
    return torch.tensor([[0.0, 0.0, -3.5, 0.0, 0.0, 0.0, 0.0, 1.0, 0.0]])


def c3(h: int = 256, w: int = 256, c: int = 64, k: int = 64):
    x = torch.rand(1, c, h, w, generator=gen(3)).half()
    wt = (torch.randn(k, c, 3, 3, generator=gen(4)) * math.sqrt(2.0 / (c * 9))).half()
    return x, wt, torch.zeros(k)


def c5(n: int = 4194304):
    x = torch.randn(n, 32, generator=gen(5)).half()
    t = torch.randn(n, 16, generator=gen(6))
    layers = kaiming_uniform_f16([(128, 32)] + [(128, 128)] * 7 + [(16, 128)], seed=7)
    return x, t, layers
