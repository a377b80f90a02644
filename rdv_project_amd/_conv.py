"""Winograd F(2x2,3x3) convolution through the C ABI (rdv_winograd3x3_*).

Two callers share this module:
  * Conv2DTensorOpWinograd3x3 (nn.py), the reference's operator
    (src/rdv/domain/nn.py:1002-1087): channels-last fp32 [H*W, CIN] in,
    [H*W, COUT] out, filter [3, 3, CIN, COUT];
  * winograd3x3_conv2d / Winograd3x3Conv2d, a build-defined NCHW functional
    form (PyTorch layouts: x [N, CIN, H, W], w [COUT, CIN, 3, 3]) for fp16
    image pipelines, with an optional fused ReLU.
There is no CPU path: without the HIP library or a GPU every call raises.
"""
from __future__ import annotations

import torch

from . import _lib
from .core import current_stream_handle, device

_DTYPES = {torch.float32: _lib.DTYPE_F32, torch.float16: _lib.DTYPE_F16}


def _dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"{what} must be float32 or float16, got {t.dtype}") from None


def conv_desc(batch: int, H: int, W: int, cin: int, cout: int, in_layout: int, in_dtype: int,
              out_layout: int, out_dtype: int, relu: bool) -> _lib.ConvDesc:
    d = _lib.ConvDesc()
    d.batch, d.H, d.W, d.cin, d.cout = batch, H, W, cin, cout
    d.in_layout, d.in_dtype, d.out_layout, d.out_dtype = in_layout, in_dtype, out_layout, out_dtype
    d.relu = 1 if relu else 0
    return d


def validate(d: _lib.ConvDesc) -> None:
    lib = _lib.load()
    _lib.check(lib.rdv_winograd3x3_validate(d), "Conv2DTensorOpWinograd3x3")


def transform_weight(w: torch.Tensor, layout: int) -> torch.Tensor:
    """U = G g G^T of every filter, packed for the kernel (a uint8 device
    buffer).  w is [3, 3, CIN, COUT] (layout RSCK) or [COUT, CIN, 3, 3] (KCRS)."""
    if layout == _lib.WLAYOUT_RSCK:
        assert w.dim() == 4 and tuple(w.shape[:2]) == (3, 3), "weight must be [3, 3, in_channels, out_channels]"
        cin, cout = int(w.shape[2]), int(w.shape[3])
    else:
        assert w.dim() == 4 and tuple(w.shape[2:]) == (3, 3), "weight must be [out_channels, in_channels, 3, 3]"
        cout, cin = int(w.shape[0]), int(w.shape[1])
    lib = _lib.load()
    nbytes = lib.rdv_winograd3x3_weight_bytes(cin, cout)
    if nbytes < 0:
        _lib.check(int(nbytes), "Conv2DTensorOpWinograd3x3")
    w = w.to(device()).contiguous()
    U = torch.empty(int(nbytes), dtype=torch.uint8, device=w.device)
    _lib.check(lib.rdv_winograd3x3_transform_weight(w.data_ptr(), layout, _dtype_code(w, "weight"), cin, cout,
                                                    U.data_ptr(), current_stream_handle()),
               "winograd weight transform")
    return U


def forward(d: _lib.ConvDesc, x: torch.Tensor, U: torch.Tensor, bias: torch.Tensor | None, y: torch.Tensor) -> None:
    """Launches the convolution on torch's current stream (asynchronous)."""
    lib = _lib.load()
    bp = None if bias is None else bias.data_ptr()
    _lib.check(lib.rdv_winograd3x3_forward(d, x.data_ptr(), U.data_ptr(), bp, y.data_ptr(), current_stream_handle()),
               "Conv2DTensorOpWinograd3x3")


class Winograd3x3Conv2d:
    """'same'-padded, stride-1 3x3 convolution of NCHW images with a fixed
    filter bank w [COUT, CIN, 3, 3] (transformed once here) and optional fp32
    bias [COUT].  Calls are asynchronous on torch's current stream."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None = None) -> None:
        assert weight.dim() == 4 and tuple(weight.shape[2:]) == (3, 3), "weight must be [COUT, CIN, 3, 3]"
        self.out_channels, self.in_channels = int(weight.shape[0]), int(weight.shape[1])
        self.U = transform_weight(weight, _lib.WLAYOUT_KCRS)
        if bias is not None:
            assert tuple(bias.shape) == (self.out_channels,), "bias must be [out_channels]"
            bias = bias.to(device=self.U.device, dtype=torch.float32).contiguous()
        self.bias = bias

    def __call__(self, x: torch.Tensor, relu: bool = False, out_dtype: torch.dtype | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
        assert x.dim() == 4 and x.is_cuda, "x must be a CUDA tensor [N, CIN, H, W]"
        n, cin, H, W = (int(s) for s in x.shape)
        assert cin == self.in_channels, f"x has {cin} channels, the filters expect {self.in_channels}"
        x = x.contiguous()
        odt = out_dtype or x.dtype
        if out is None:
            out = torch.empty((n, self.out_channels, H, W), dtype=odt, device=x.device)
        else:
            if not isinstance(out, torch.Tensor) or out.device.type != "cuda" or out.device != x.device:
                raise TypeError(f"out must be a GPU tensor on {x.device}")
            assert out.is_contiguous() and tuple(out.shape) == (n, self.out_channels, H, W) and out.dtype == odt
        d = conv_desc(n, H, W, cin, self.out_channels, _lib.LAYOUT_CHW, _dtype_code(x, "x"), _lib.LAYOUT_CHW,
                      _dtype_code(out, "out"), relu)
        forward(d, x, self.U, self.bias, out)
        return out


def winograd3x3_conv2d(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
                       relu: bool = False, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """One-shot form of Winograd3x3Conv2d (transforms the filters every call)."""
    return Winograd3x3Conv2d(weight, bias)(x, relu=relu, out_dtype=out_dtype)
