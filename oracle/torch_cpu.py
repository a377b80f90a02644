"""torch-CPU restatement of the hot path — TEST INFRASTRUCTURE ONLY (see
oracle/__init__.py).  bench.py times these functions as its CPU baseline
(`cpu_baseline`, kind "port"); tests/test_oracle_torch_cpu.py checks them
against the numpy oracle, which is what pins them.

The reference itself cannot run here or on the GPU box (it needs the vulky
package and a Vulkan device), so the baseline is this repository's
own CPU statement of the same arithmetic, written the way a CPU user of torch
would: fp32 GEMMs on fp16-rounded operands (LinearFast,
src/rdv/shaders/maps/linear_fast.h:61-98: operands staged as float16, fp32
accumulation, fp32 bias after), torch's fp32 direct convolution for the 3x3
conv, vectorised front-to-back compositing, and torch autograd for the
training step.  Every function runs under the caller's torch.set_num_threads.
"""
from __future__ import annotations

import math

import torch


def _f16(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float16).to(torch.float32)


def freq_encode(p: torch.Tensor, octaves: int, width: int | None = None) -> torch.Tensor:
    """[p, sin(2^k pi p), cos(2^k pi p) for k < octaves], zero padded (build-defined)."""
    feats = [p]
    for k in range(octaves):
        t = p * (math.pi * 2.0 ** k)
        feats += [torch.sin(t), torch.cos(t)]
    out = torch.cat(feats, dim=-1)
    if width is not None and width > out.shape[-1]:
        out = torch.nn.functional.pad(out, (0, width - out.shape[-1]))
    return out


_ACTS = {
    "none": lambda v: v,
    "relu": torch.relu,
    "softplus": torch.nn.functional.softplus,
    "sigmoid": torch.sigmoid,
}


def pack_layers(layers):
    """fp16-rounded fp32 weights (transposed for x @ W^T) and fp32 biases, prepared once
    as a CPU user would keep them."""
    return [(_f16(torch.as_tensor(w, dtype=torch.float32)).t().contiguous(), torch.as_tensor(b, dtype=torch.float32))
            for w, b in layers]


def mlp_forward(x: torch.Tensor, packed, acts, encoding: tuple | None = None) -> torch.Tensor:
    """LinearFast chain on every row: fp16-rounded layer inputs and weights,
    fp32 matmul, fp32 bias, activation (full-workgroup numerics)."""
    h = freq_encode(x, *encoding) if encoding is not None else x
    for (wt, b), a in zip(packed, acts):
        h = _ACTS[a](torch.addmm(b, _f16(h), wt))
    return h


def conv3x3(x: torch.Tensor, w: torch.Tensor, relu: bool = True) -> torch.Tensor:
    """'same'-padded stride-1 3x3 convolution in fp32 on fp16-valued NCHW input
    and OIHW filters (the direct-conv equivalent of the Winograd op)."""
    y = torch.nn.functional.conv2d(x, w, padding=1)
    return torch.relu(y) if relu else y


def render_ea(rays: torch.Tensor, packed, samples: int) -> torch.Tensor:
    """Emission-absorption colour [N, 3] of rays [N, 6] = (o, w) through
    [-1,1]^3: samples t_i = t0 + (i + 1/2) dt, field (3 -> ... -> 4, ReLU hidden,
    raw head), sigma = softplus, c = sigmoid, front-to-back compositing."""
    o, w = rays[:, 0:3], rays[:, 3:6]
    inv = 1.0 / w
    xc, s = -o * inv, inv.abs()
    tmin = (xc - s).max(dim=1).values
    tmax = (xc + s).min(dim=1).values
    hit = ~((tmax <= 0) | (tmin > tmax))
    t0 = tmin.clamp_min(0.0)
    dt = torch.where(hit, (tmax - t0) / samples, torch.zeros_like(t0))
    t = t0[:, None] + (torch.arange(samples, dtype=torch.float32)[None, :] + 0.5) * dt[:, None]
    p = (o[:, None, :] + t[..., None] * w[:, None, :]).reshape(-1, 3)
    acts = ["relu"] * (len(packed) - 1) + ["none"]
    f = mlp_forward(p, packed, acts).reshape(-1, samples, 4)
    a = torch.nn.functional.softplus(f[..., 0]) * dt[:, None]
    excl = torch.cumsum(a, dim=1) - a
    wgt = torch.exp(-excl) * (1.0 - torch.exp(-a))
    return (wgt[..., None] * torch.sigmoid(f[..., 1:4])).sum(dim=1)


def train_step(x: torch.Tensor, target: torch.Tensor, params):
    """Forward (LinearFast chain, ReLU hidden, linear head), MSE loss and
    autograd backward in fp32.  params: [(W, b)] fp32 leaf tensors with
    requires_grad; returns the loss and leaves the gradients in .grad."""
    h = x
    for i, (w, b) in enumerate(params):
        h = torch.addmm(b, _f16(h), _f16(w).t())
        if i + 1 < len(params):
            h = torch.relu(h)
    loss = torch.mean((h - target) ** 2)
    for w, b in params:
        w.grad = None
        b.grad = None
    loss.backward()
    return loss
