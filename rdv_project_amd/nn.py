"""Small-network nodes of the rdv API (reference: src/rdv/domain/nn.py).

Map nodes compose with `>>` and are evaluated by the fused HIP MLP kernels:
  Linear / LinearFast / linear   nn.py:25-104
  ReLU / relu                    nn.py:107-119
Build-defined additions (no reference counterpart, needed by the benchmark
configurations): FrequencyEncoding, Softplus, Sigmoid, DensityRGB.
"""
from __future__ import annotations

import torch

from . import _lib
from .core import RDVObject, wrap
from .maths import Map


class _LinearBase(Map):
    """weight [out_features, in_features] (PyTorch nn.Linear layout), bias
    [out_features], both fp32 (reference: _LinearBase, nn.py:25-54)."""

    _precision = _lib.PREC_F32
    __next_id__ = 0

    def __init__(self, weight, bias) -> None:
        weight = weight if isinstance(weight, RDVObject) else wrap(_float32(weight))
        bias = bias if isinstance(bias, RDVObject) else wrap(_float32(bias))
        assert len(weight.shape) == 2, "weight must be [out_features, in_features]"
        out_features, in_features = weight.shape
        assert tuple(bias.shape) == (out_features,), "bias must be [out_features]"
        if weight.scalar_type != torch.float32 or bias.scalar_type != torch.float32:
            raise TypeError("weight and bias must be float32 buffers (reference fields are Buffer[FLOAT32])")
        self.IN = int(in_features)
        self.OUT = int(out_features)
        self.weight = weight
        self.bias = bias
        cls = type(self)
        self.id = cls.__next_id__
        cls.__next_id__ += 1


def _float32(t):
    t = torch.as_tensor(t)
    return t.to(torch.float32) if t.is_floating_point() and t.dtype != torch.float32 else t


class Linear(_LinearBase):
    """y = W @ x + b in exact fp32 (reference: nn.py:57-74, shaders/maps/linear.h)."""

    _precision = _lib.PREC_F32
    __next_id__ = 0


class LinearFast(_LinearBase):
    """y = W @ x + b on the fp16 matrix cores with fp32 accumulation
    (reference: nn.py:77-96, shaders/maps/linear_fast.h)."""

    _precision = _lib.PREC_F16
    __next_id__ = 0


def linear(weight, bias, f16: bool = False) -> _LinearBase:
    """Linear (exact fp32) or, with f16=True, LinearFast (reference: nn.py:99-104)."""
    return (LinearFast if f16 else Linear)(weight, bias)


class _Activation(Map):
    """Elementwise map; generic in width until composed."""

    _act = _lib.ACT_NONE
    _shape_preserving = True


class ReLU(_Activation):
    """f(x) = max(x, 0) (reference: nn.py:107-116, shaders/maps/relu.h)."""

    _act = _lib.ACT_RELU


relu = ReLU()


class Softplus(_Activation):
    """f(x) = log(1 + exp(x)) (build-defined)."""

    _act = _lib.ACT_SOFTPLUS


softplus = Softplus()


class Sigmoid(_Activation):
    """f(x) = 1 / (1 + exp(-x)) (build-defined)."""

    _act = _lib.ACT_SIGMOID


sigmoid = Sigmoid()


class DensityRGB(_Activation):
    """Radiance-field head (build-defined): softplus on channel 0 (density),
    sigmoid on the remaining channels (colour)."""

    _act = _lib.ACT_DENSITY_RGB


density_rgb = DensityRGB()


class FrequencyEncoding(Map):
    """gamma(p) = [p, sin(2^k pi p), cos(2^k pi p) for k < octaves], zero padded
    to `pad_to` features (build-defined; NeRF-style positional encoding).

    Feature order: p_0..p_{D-1}, then for each octave k the D sines followed by
    the D cosines."""

    def __init__(self, in_features: int = 3, octaves: int = 6, pad_to: int | None = None) -> None:
        assert in_features >= 1 and octaves >= 1
        width = in_features * (1 + 2 * octaves)
        if pad_to is not None:
            assert pad_to >= width, f"pad_to ({pad_to}) is smaller than the encoded width ({width})"
            width = pad_to
        self.in_features = int(in_features)
        self.octaves = int(octaves)
        self.IN = self.in_features
        self.OUT = int(width)
