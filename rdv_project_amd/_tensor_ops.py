"""Linear, ReLU and data-movement tensor operations through the C ABI
(rdv_linear_op, rdv_relu_op, rdv_downsample2x, rdv_upsample2x,
rdv_concat_channels): descriptor building, weight preparation and launches
for the TensorOperation classes of nn.py.  There is no CPU path: without the HIP
library or a GPU every launch raises."""
from __future__ import annotations

import ctypes as C

import torch

from . import _lib
from .core import current_stream_handle


def linear_desc(rows: int, in_features: int, out_features: int, precision: int, wkind: int,
                relu: bool = False) -> _lib.LinearOpDesc:
    d = _lib.LinearOpDesc()
    d.rows, d.in_features, d.out_features = int(rows), int(in_features), int(out_features)
    d.precision, d.wkind, d.relu, d.reserved = int(precision), int(wkind), 1 if relu else 0, 0
    return d


def validate(d: _lib.LinearOpDesc, what: str) -> None:
    _lib.check(_lib.load().rdv_linear_op_validate(C.byref(d)), what)


def _aligned(t: torch.Tensor, nbytes: int = 16) -> torch.Tensor:
    """t itself when its data pointer is nbytes-aligned, else an aligned copy."""
    return t if t.data_ptr() % nbytes == 0 else t.clone()


def linear(d: _lib.LinearOpDesc, x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, y: torch.Tensor,
           what: str) -> None:
    """y = x W^T + b per descriptor d (x, b, y fp32 device tensors)."""
    x = _aligned(x.contiguous())
    if d.wkind != _lib.WKIND_F16_TILED16:
        w = _aligned(w.contiguous())
    assert y.is_contiguous() and y.data_ptr() % 16 == 0, "result buffer must be contiguous and 16-byte aligned"
    _lib.check(_lib.load().rdv_linear_op(C.byref(d), C.c_void_p(x.data_ptr()), C.c_void_p(w.data_ptr()),
                                         C.c_void_p(b.contiguous().data_ptr()), C.c_void_p(y.data_ptr()),
                                         C.c_void_p(current_stream_handle())), what)


def relu(x: torch.Tensor, y: torch.Tensor) -> None:
    """y = max(x, 0) elementwise (fp32 device tensors of equal size)."""
    x = _aligned(x.contiguous())
    assert y.is_contiguous() and y.data_ptr() % 16 == 0 and y.numel() == x.numel()
    _lib.check(_lib.load().rdv_relu_op(C.c_void_p(x.data_ptr()), C.c_void_p(y.data_ptr()), C.c_int64(x.numel()),
                                       C.c_void_p(current_stream_handle())), "ReLUTensorOp")


def conv2d_desc(H: int, W: int, cin: int, cout: int, kh: int, kw: int, precision: int, w_layout: int,
                relu: bool = False) -> _lib.Conv2dDesc:
    d = _lib.Conv2dDesc()
    d.H, d.W, d.cin, d.cout, d.kh, d.kw = int(H), int(W), int(cin), int(cout), int(kh), int(kw)
    d.precision, d.w_layout, d.relu, d.reserved = int(precision), int(w_layout), 1 if relu else 0, 0
    return d


def conv2d_validate(d: _lib.Conv2dDesc, what: str) -> None:
    _lib.check(_lib.load().rdv_conv2d_validate(C.byref(d)), what)


def conv2d(d: _lib.Conv2dDesc, x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, y: torch.Tensor,
           what: str) -> None:
    """y = conv(x, w) + b per descriptor d (fp32 device tensors; w read at every call)."""
    x = _aligned(x.contiguous())
    _out_buffer(y)
    w = w.contiguous()
    bp = 0 if b is None else b.contiguous().data_ptr()
    _lib.check(_lib.load().rdv_conv2d(C.byref(d), C.c_void_p(x.data_ptr()), C.c_void_p(w.data_ptr()),
                                      C.c_void_p(bp), C.c_void_p(y.data_ptr()),
                                      C.c_void_p(current_stream_handle())), what)


def _out_buffer(y: torch.Tensor) -> None:
    assert y.is_contiguous() and y.data_ptr() % 16 == 0, "result buffer must be contiguous and 16-byte aligned"


def downsample2x(x: torch.Tensor, H: int, W: int, y: torch.Tensor) -> None:
    """y[(H/2)(W/2), C] = 2x2 average pool of x[H W, C] (fp32 device tensors)."""
    x = _aligned(x.contiguous())
    _out_buffer(y)
    _lib.check(_lib.load().rdv_downsample2x(C.c_void_p(x.data_ptr()), C.c_int64(H), C.c_int64(W),
                                            C.c_int32(int(x.shape[1])), C.c_void_p(y.data_ptr()),
                                            C.c_void_p(current_stream_handle())), "Downsample2xTensorOp")


def upsample2x(x: torch.Tensor, H: int, W: int, y: torch.Tensor) -> None:
    """y[(2H)(2W), C] = nearest-neighbour 2x upsample of x[H W, C]."""
    x = _aligned(x.contiguous())
    _out_buffer(y)
    _lib.check(_lib.load().rdv_upsample2x(C.c_void_p(x.data_ptr()), C.c_int64(H), C.c_int64(W),
                                          C.c_int32(int(x.shape[1])), C.c_void_p(y.data_ptr()),
                                          C.c_void_p(current_stream_handle())), "Upsample2xTensorOp")


def concat(x1: torch.Tensor, x2: torch.Tensor, y: torch.Tensor) -> None:
    """y[rows, C1 + C2] = [x1 | x2]."""
    x1 = _aligned(x1.contiguous())
    x2 = _aligned(x2.contiguous())
    _out_buffer(y)
    _lib.check(_lib.load().rdv_concat_channels(C.c_void_p(x1.data_ptr()), C.c_int32(int(x1.shape[1])),
                                               C.c_void_p(x2.data_ptr()), C.c_int32(int(x2.shape[1])),
                                               C.c_int64(int(x1.shape[0])), C.c_void_p(y.data_ptr()),
                                               C.c_void_p(current_stream_handle())), "ConcatTensorOp")


def tile_weight_fp16(w: torch.Tensor) -> torch.Tensor:
    """[out, in] -> flat fp16 [out/16][in/16][16 k][16 n] tiles, the layout of
    LinearTensorOpFast's weight_tiled (reference: _tile_weight_fp16,
    src/rdv/domain/nn.py:472-490)."""
    out_features, in_features = int(w.shape[0]), int(w.shape[1])
    t = w.reshape(out_features // 16, 16, in_features // 16, 16).permute(0, 2, 3, 1)
    return t.to(torch.float16).contiguous().reshape(-1)


def cast_fp16(w: torch.Tensor) -> torch.Tensor:
    """fp16 copy, same [out, in] layout (reference: _cast_fp16, nn.py:493-501)."""
    return w.to(torch.float16).contiguous()


def max_subgroups(fixed_bytes: int, per_subgroup_bytes: int, divides, budget: int = 49152, cap: int = 32) -> int:
    """The reference's subgroups-per-workgroup choice (nn.py:504-519): the
    largest power of two s <= cap with fixed + s * per_subgroup <= budget and
    divides(s).  It decides only which shapes LinearTensorOpSimple accepts
    and the SPT attribute; the HIP kernel's tiling does not depend on it."""
    spt = 1
    while spt * 2 <= cap and fixed_bytes + spt * 2 * per_subgroup_bytes <= budget and divides(spt * 2):
        spt *= 2
    return spt
