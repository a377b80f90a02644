"""MLP training step through the C ABI (rdv_mlp_train_step): forward, MSE loss
and backward of a LinearFast / ReLU chain with fp32 weight gradients
(build-defined: the reference has no backward pass)."""
from __future__ import annotations

import ctypes as C

import torch

from . import _chain, _lib
from .core import current_stream_handle, device, launch_scope
from .maths import Map

_WS: dict = {}


def _workspace(key, nbytes: int) -> torch.Tensor:
    hit = _WS.get(key)
    if hit is not None and hit.numel() >= nbytes:
        return hit
    buf = torch.empty(int(nbytes) + 256, dtype=torch.uint8, device=device())
    off = (-buf.data_ptr()) % 256
    buf = buf[off: off + int(nbytes)]
    _WS.clear()  # one workspace at a time: these are large
    _WS[key] = buf
    return buf


def _check_grads(grads, layers) -> None:
    """Caller-supplied gradient buffers must be exactly what the kernels write:
    one (dW, db) pair per layer, contiguous fp32 GPU tensors of shape [OUT, IN]
    and [OUT].  Checked before anything is launched."""
    if not isinstance(grads, (list, tuple)) or len(grads) != len(layers):
        raise TypeError(f"grads must be a list of {len(layers)} (dW, db) pairs, one per layer")
    for i, (pair, lay) in enumerate(zip(grads, layers)):
        if not isinstance(pair, (list, tuple)) or len(pair) != 2:
            raise TypeError(f"grads[{i}] must be a (dW, db) pair")
        for t, shape, what in ((pair[0], (lay.OUT, lay.IN), "dW"), (pair[1], (lay.OUT,), "db")):
            if not isinstance(t, torch.Tensor):
                raise TypeError(f"grads[{i}] {what} must be a torch tensor")
            if t.dtype != torch.float32:
                raise TypeError(f"grads[{i}] {what} must be float32, got {t.dtype}")
            if tuple(t.shape) != shape:
                raise TypeError(f"grads[{i}] {what} must have shape {list(shape)}, got {list(t.shape)}")
            if not t.is_contiguous():
                raise TypeError(f"grads[{i}] {what} must be contiguous")
            if t.device.type != "cuda":
                raise TypeError(f"grads[{i}] {what} must be a GPU tensor, got device {t.device}")


def mse_backward(m: Map, x, target, grads=None, loss=None):
    """Loss and gradients of mean((m(x) - target)^2) with respect to every
    layer's weight and bias.  x: [n, in] (fp16, or fp32 rounded to fp16 as
    LinearFast does), target: [n, out] fp32.  Returns (loss, [(dW, db), ...])
    with a 0-d fp32 loss tensor and fp32 dW [out, in] and db [out] per layer,
    in chain order.  Every call returns fresh tensors unless the caller passes
    them: `grads` (contiguous fp32 GPU tensors of exactly those shapes) and
    `loss` (a 0-d or 1-element contiguous fp32 GPU tensor), else TypeError.
    Passing both makes a steady-state call allocate nothing."""
    xt = torch.as_tensor(x)
    tt = torch.as_tensor(target)
    assert xt.dim() == 2 and tt.dim() == 2 and xt.shape[0] == tt.shape[0], "x [n, in] and target [n, out]"
    n = int(xt.shape[0])
    p = _chain.plan_chain(m, int(xt.shape[1]))
    assert tt.shape[1] == p.out_features, f"target has {tt.shape[1]} columns, the chain outputs {p.out_features}"
    if grads is not None:
        _check_grads(grads, p.layers)
    if loss is not None:
        _check_loss(loss)
    packed = _chain.packed_params(m, p)
    xh = xt.to(device=device(), dtype=torch.float16).contiguous()
    th = tt.to(device=device(), dtype=torch.float32).contiguous()
    lib = _lib.load()
    nbytes = lib.rdv_mlp_train_workspace_bytes(C.byref(p.desc), C.c_int64(n))
    if nbytes < 0:
        _lib.check(int(nbytes), "mse_backward")
    ws = _workspace((p.signature, n), int(nbytes))
    if grads is None:
        grads = [(torch.empty(l.OUT, l.IN, dtype=torch.float32, device=device()),
                  torch.empty(l.OUT, dtype=torch.float32, device=device())) for l in p.layers]
    if loss is None:
        loss = torch.empty((), dtype=torch.float32, device=device())
    dws = _lib.void_ptr_array([g[0].data_ptr() for g in grads])
    dbs = _lib.void_ptr_array([g[1].data_ptr() for g in grads])
    with launch_scope():
        _lib.check(lib.rdv_mlp_train_step(C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.c_void_p(xh.data_ptr()),
                                          C.c_void_p(th.data_ptr()), C.c_int64(n), C.c_void_p(ws.data_ptr()),
                                          C.c_int64(ws.numel()), C.c_void_p(loss.data_ptr()), dws, dbs,
                                          C.c_void_p(current_stream_handle())), "mse_backward")
    return loss, grads


def _check_loss(loss) -> None:
    """A caller-supplied loss buffer: one contiguous fp32 element on the GPU."""
    if not isinstance(loss, torch.Tensor):
        raise TypeError("loss must be a torch tensor")
    if loss.dtype != torch.float32 or loss.numel() != 1 or not loss.is_contiguous():
        raise TypeError(f"loss must be one contiguous float32 element, got {loss.dtype} {list(loss.shape)}")
    if loss.device.type != "cuda":
        raise TypeError(f"loss must be a GPU tensor, got device {loss.device}")
