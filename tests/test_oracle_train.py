"""Pins oracle/train.py against torch autograd (float64, fp16 casts as
straight-through), a finite difference, and a planted mistake (CPU only)."""
import numpy as np
import pytest
import torch

from oracle import train as T


def _layers(dims, seed):
    g = np.random.default_rng(seed)
    out = []
    for i in range(len(dims) - 1):
        lim = np.sqrt(6.0 / dims[i])
        W = g.uniform(-lim, lim, (dims[i + 1], dims[i])).astype(np.float16).astype(np.float32)
        b = g.normal(0, 0.1, dims[i + 1]).astype(np.float32)
        out.append((W, b))
    return out


def _torch_grads(x, layers, target):
    h = torch.tensor(x, dtype=torch.float64).half().double()
    params = []
    for i, (W, b) in enumerate(layers):
        Wt = torch.tensor(W, dtype=torch.float64, requires_grad=True)
        bt = torch.tensor(b, dtype=torch.float64, requires_grad=True)
        params.append((Wt, bt))
        z = h @ Wt.half().double().T + bt
        h = torch.relu(z).half().double() if i + 1 < len(layers) else z
    loss = torch.mean((h - torch.tensor(target, dtype=torch.float64)) ** 2)
    loss.backward()
    return loss.item(), [(W.grad.numpy(), b.grad.numpy()) for W, b in params]


@pytest.mark.parametrize("dims", [[32, 128, 128, 16], [16, 64, 32, 8], [32, 128, 128, 128, 128, 16]])
def test_matches_torch_autograd(dims):
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (257, dims[0])).astype(np.float32)
    t = rng.normal(0, 1, (257, dims[-1])).astype(np.float32)
    layers = _layers(dims, 2)
    loss, grads = T.mse_grads(x, layers, t)
    tl, tg = _torch_grads(x, layers, t)
    assert abs(loss - tl) <= 1e-6 * abs(tl)
    for (dw, db), (rw, rb) in zip(grads, tg):
        # the oracle rounds each layer's sum to fp32 before fp16 (as LinearFast does), torch
        # rounds float64 to fp16 once: rare 1-ulp activation differences, so compare per layer
        assert np.linalg.norm(dw - rw) <= 1e-3 * np.linalg.norm(rw)
        assert np.linalg.norm(db - rb) <= 1e-3 * np.linalg.norm(rb)


def test_finite_difference_of_a_bias():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (64, 16)).astype(np.float32)
    t = rng.normal(0, 1, (64, 8)).astype(np.float32)
    layers = _layers([16, 32, 8], 4)
    _, grads = T.mse_grads(x, layers, t)
    # the head's bias enters y linearly (no fp16 rounding after it): central difference is exact up to fp32 noise
    eps = 1e-2
    for k in range(3):
        lp = [(W, b.copy()) for W, b in layers]
        lm = [(W, b.copy()) for W, b in layers]
        lp[-1][1][k] += eps
        lm[-1][1][k] -= eps
        fd = (T.mse_grads(x, lp, t)[0] - T.mse_grads(x, lm, t)[0]) / (2 * eps)
        assert abs(fd - grads[-1][1][k]) <= 1e-4 * max(1.0, abs(fd))


def test_planted_mistake_is_caught(monkeypatch):
    """Forgetting the ReLU mask in the backward breaks agreement with autograd."""
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (128, 16)).astype(np.float32)
    t = rng.normal(0, 1, (128, 8)).astype(np.float32)
    layers = _layers([16, 32, 32, 8], 6)
    real = T.mse_grads
    def bad(x, layers, target):
        hs, y = T.forward_states(x, layers)
        tt = np.asarray(target, np.float64)
        n, out = y.shape
        dz = 2.0 * (y - tt) / (n * out)
        grads = [None] * len(layers)
        for l in range(len(layers) - 1, -1, -1):
            W = np.asarray(layers[l][0], np.float64)
            grads[l] = (dz.T @ hs[l], dz.sum(axis=0))
            if l > 0:
                dz = dz @ W
        return np.mean((y - tt) ** 2), grads
    monkeypatch.setattr(T, "mse_grads", bad)
    _, g_bad = T.mse_grads(x, layers, t)
    _, g_ref = _torch_grads(x, layers, t)
    assert np.abs(g_bad[0][0] - g_ref[0][0]).max() > 1e-3 * np.abs(g_ref[0][0]).max()
    monkeypatch.setattr(T, "mse_grads", real)
