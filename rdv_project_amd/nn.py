"""Small-network nodes of the rdv API (reference: src/rdv/domain/nn.py).

Map nodes compose with `>>` and are evaluated by the fused HIP MLP kernels:
  Linear / LinearFast / linear   nn.py:25-104
  ReLU / relu                    nn.py:107-119
TensorOperation nodes dispatch eagerly, one kernel per op:
  ReLUTensorOp                   nn.py:362-374
  LinearTensorOp                 nn.py:377-411
  LinearTensorOpFast             nn.py:541-605
  LinearTensorOpMine             nn.py:1153-1201
  LinearTensorOpSimple           nn.py:1204-1300
  LinearTensorOpSmall            nn.py:1303-1411
  Conv2DTensorOp                 nn.py:414-470
  Conv2DTensorOpFast             nn.py:608-668
  Conv2DTensorOpSimple           nn.py:669-756
  Conv2DTensorOpSimple3x3        nn.py:757-850
  Conv2DTensorOpWindow3x3        nn.py:851-1000
  Conv2DTensorOpWinograd3x3      nn.py:1002-1087
  Downsample2xTensorOp           nn.py:1090-1107
  Upsample2xTensorOp             nn.py:1110-1125
  ConcatTensorOp                 nn.py:1128-1150
Build-defined additions (no reference counterpart, needed by the benchmark
configurations): FrequencyEncoding, Softplus, Sigmoid, DensityRGB.
"""
from __future__ import annotations

import torch

from . import _conv, _lib, _tensor_ops
from .core import RDVObject, wrap
from .maths import Map, TensorOperation, _as_op_input


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


# ============================================================ TENSOR OPERATIONS


def _op_float32(data: RDVObject, what: str) -> RDVObject:
    """The reference binds these inputs as Buffer[FLOAT32]; other float
    buffers are converted (a copy, so later in-place updates of the original
    are not seen)."""
    if data.scalar_type == torch.float32:
        return data
    if not data.scalar_type.is_floating_point:
        raise TypeError(f"{what} must be a floating-point buffer, got {data.scalar_type}")
    return wrap(data.as_tensor("torch").to(torch.float32))


class ReLUTensorOp(TensorOperation):
    """f(x) = max(x, 0), elementwise (reference: nn.py:362-374,
    shaders/tensors/relu_tensor_op.h:3-22).  x may be another TensorOperation
    or raw data; a NaN input gives 0."""

    def __init__(self, x) -> None:
        data, shape, upstream = _as_op_input(x)
        self.x_buf = _op_float32(data, "x")
        self._upstream = upstream
        super().__init__(shape)

    def _forward(self) -> None:
        _tensor_ops.relu(self.x_buf.as_tensor("torch"), self._result_t)


class _LinearTensorOpBase(TensorOperation):
    """y = x W^T + b for x [batch, in_features], weight [out_features,
    in_features] (PyTorch nn.Linear layout), bias [out_features]; result
    [batch, out_features] fp32.  Shared argument handling of the reference's
    linear tensor ops (nn.py:377-411, 541-605, 1153-1411)."""

    _precision = _lib.PREC_F16
    _wkind = _lib.WKIND_F32

    def _bind(self, x, weight, bias):
        name = type(self).__name__
        data, shape, upstream = _as_op_input(x)
        assert len(shape) == 2, f"{name} requires a 2D (BATCH, in_features) input"
        batch, in_features = shape
        weight = weight if isinstance(weight, RDVObject) else wrap(weight)
        bias = bias if isinstance(bias, RDVObject) else wrap(bias)
        assert len(weight.shape) == 2, "weight must be [out_features, in_features]"
        out_features, weight_in_features = weight.shape
        assert weight_in_features == in_features, "weight's own in_features must match x's own trailing dim"
        assert tuple(bias.shape) == (out_features,), "bias must be [out_features]"
        self.x_buf = _op_float32(data, "x")
        self.bias = _op_float32(bias, "bias")
        self._upstream = upstream
        self.INF, self.OUTF = int(in_features), int(out_features)
        return int(batch), int(in_features), int(out_features), weight

    def _finish(self, batch: int) -> None:
        self._desc = _tensor_ops.linear_desc(batch, self.INF, self.OUTF, self._precision, self._wkind)
        _tensor_ops.validate(self._desc, type(self).__name__)
        super().__init__([batch, self.OUTF])

    def _weight_buffer(self) -> torch.Tensor:
        return self.weight.as_tensor("torch")

    def _forward(self) -> None:
        _tensor_ops.linear(self._desc, self.x_buf.as_tensor("torch"), self._weight_buffer(),
                           self.bias.as_tensor("torch"), self._result_t, type(self).__name__)


class LinearTensorOp(_LinearTensorOpBase):
    """y = W @ x + b in fp32 (reference: nn.py:377-411,
    shaders/tensors/linear_tensor_op.h:8-51).  batch must be a multiple of 4,
    in_features and out_features multiples of 8.  The fp32 weight is read at
    every dispatch, so in-place updates of it are seen by evaluate()."""

    _precision = _lib.PREC_F32
    _wkind = _lib.WKIND_F32

    def __init__(self, x, weight, bias) -> None:
        batch, in_features, out_features, weight = self._bind(x, weight, bias)
        assert in_features % 8 == 0, f"in_features ({in_features}) must be a multiple of 8"
        assert out_features % 8 == 0, f"out_features ({out_features}) must be a multiple of 8"
        self.weight = _op_float32(weight, "weight")
        self._finish(batch)


class LinearTensorOpSmall(_LinearTensorOpBase):
    """y = W @ x + b with x and W rounded to fp16 and fp32 accumulation
    (reference: nn.py:1303-1411, shaders/tensors/linear_tensor_op_small.h:50-247).
    batch must be a multiple of 32, in_features and out_features multiples of
    16 and at most 128.  The fp32 weight is read (and rounded) at every
    dispatch.  SPT is the reference's subgroups-per-workgroup choice; the HIP
    kernel stages the whole weight block in LDS regardless."""

    _TILE_ROWS = 32
    _TILE_COLS = 16

    def __init__(self, x, weight, bias) -> None:
        batch, in_features, out_features, weight = self._bind(x, weight, bias)
        assert batch % 32 == 0, f"batch ({batch}) must be a multiple of 32"
        assert in_features % 16 == 0, f"in_features ({in_features}) must be a multiple of 16"
        assert out_features % 16 == 0, f"out_features ({out_features}) must be a multiple of 16"
        assert in_features <= 128, f"in_features ({in_features}) must be at most 128 (see this op's own docstring)"
        assert out_features <= 128, f"out_features ({out_features}) must be at most 128 (see this op's own docstring)"
        self.SPT = _tensor_ops.max_subgroups(fixed_bytes=out_features * in_features * 2,
                                             per_subgroup_bytes=32 * in_features * 2,
                                             divides=lambda s: batch % (32 * s) == 0)
        self.weight = _op_float32(weight, "weight")
        self._finish(batch)


class LinearTensorOpSimple(_LinearTensorOpBase):
    """y = W @ x + b with x and W rounded to fp16 and fp32 accumulation
    (reference: nn.py:1204-1300, shaders/tensors/linear_tensor_op_simple.h:49-116).
    batch must be a multiple of 32, in_features a multiple of 16 and
    out_features a multiple of 16 * SPT.  The weight is cast to fp16 once, at
    construction (_cast_fp16, nn.py:493-501)."""

    _TILE_ROWS = 32
    _TILE_COLS = 16
    _wkind = _lib.WKIND_F16

    def __init__(self, x, weight, bias) -> None:
        batch, in_features, out_features, weight = self._bind(x, weight, bias)
        assert batch % 32 == 0, f"batch ({batch}) must be a multiple of 32"
        assert in_features % 16 == 0, f"in_features ({in_features}) must be a multiple of 16"
        spt = _tensor_ops.max_subgroups(fixed_bytes=32 * in_features * 2,
                                        per_subgroup_bytes=16 * in_features * 2,
                                        divides=lambda s: out_features % (16 * s) == 0)
        out_tile = 16 * spt
        assert out_features % out_tile == 0, f"out_features ({out_features}) must be a multiple of {out_tile}"
        self.SPT = spt
        self.weight = wrap(_tensor_ops.cast_fp16(weight.as_tensor("torch")))
        self._finish(batch)


class LinearTensorOpFast(_LinearTensorOpBase):
    """y = W @ x + b with x and W rounded to fp16 and fp32 accumulation
    (reference: nn.py:541-605, shaders/tensors/linear_tensor_op_fast.h:37-122).
    batch must be a multiple of 64, in_features a multiple of 16, out_features a
    multiple of 32.  The weight is rearranged once, at construction, into the
    reference's fp16 tile layout weight_tiled (_tile_weight_fp16,
    nn.py:472-490), which the kernel reads directly."""

    _TILE_ROWS = 64
    _TILE_COLS = 32
    _wkind = _lib.WKIND_F16_TILED16

    def __init__(self, x, weight, bias) -> None:
        batch, in_features, out_features, weight = self._bind(x, weight, bias)
        assert batch % 64 == 0, f"batch ({batch}) must be a multiple of 64"
        assert in_features % 16 == 0, f"in_features ({in_features}) must be a multiple of 16"
        assert out_features % 32 == 0, f"out_features ({out_features}) must be a multiple of 32"
        self.weight_tiled = wrap(_tensor_ops.tile_weight_fp16(weight.as_tensor("torch")))
        self._finish(batch)

    def _weight_buffer(self) -> torch.Tensor:
        return self.weight_tiled.as_tensor("torch")


class LinearTensorOpMine(_LinearTensorOpBase):
    """y = W @ x + b with x and W rounded to fp16 and fp32 accumulation
    (reference: nn.py:1153-1201, shaders/tensors/linear_tensor_op_mine.h:51-133).
    batch must be a multiple of 32, in_features and out_features multiples of
    16.  The fp32 weight is read (and rounded) at every dispatch."""

    _TILE_ROWS = 32
    _TILE_COLS = 16

    def __init__(self, x, weight, bias) -> None:
        batch, in_features, out_features, weight = self._bind(x, weight, bias)
        assert batch % 32 == 0, f"batch ({batch}) must be a multiple of 32"
        assert in_features % 16 == 0, f"in_features ({in_features}) must be a multiple of 16"
        assert out_features % 16 == 0, f"out_features ({out_features}) must be a multiple of 16"
        self.weight = _op_float32(weight, "weight")
        self._finish(batch)


class Conv2DTensorOpWinograd3x3(TensorOperation):
    """'same'-padded (zero border), stride-1 3x3 convolution via Winograd
    F(2x2, 3x3) (reference: nn.py:1002-1087,
    shaders/tensors/conv2d_tensor_op_winograd3x3.h).

    x: [H*W, in_channels] channels-last (a buffer or an upstream
    TensorOperation), weight: [3, 3, in_channels, out_channels], bias:
    [out_channels] fp32.  result: [H*W, out_channels] fp32.  The filters are
    transformed once, at construction (U = G g G^T in fp32, rounded to fp16,
    nn.py:522-538); per 2x2 output tile the 4x4 input patch is transformed
    (V = B^T d B, rounded to fp16), the 16 channel reductions accumulate in
    fp32 and Y = A^T M A + bias.

    Shape rules follow the reference (H, W even; channels multiples of 16)
    except for its shared-memory limits (in/out channels <= 48 and
    (H/2)(W/2) % 32 == 0, nn.py:1066-1078), which this kernel does not have:
    in_channels may be up to 64 and out_channels up to 1024."""

    _TILE_ROWS = 1
    _TILE_COLS = 16

    def __init__(self, x, weight, bias, H: int, W: int) -> None:
        data, shape, upstream = _as_op_input(x)
        assert len(shape) == 2, "Conv2DTensorOpWinograd3x3 requires a 2D (H*W, in_channels) input"
        hw, in_channels = shape
        assert hw == H * W, f"H*W ({H * W}) must match x's own row count ({hw})"
        weight = weight if isinstance(weight, RDVObject) else wrap(weight)
        bias = bias if isinstance(bias, RDVObject) else wrap(_float32(bias))
        assert tuple(weight.shape[:2]) == (3, 3), "weight must be [3, 3, in_channels, out_channels]"
        _, _, weight_in_channels, out_channels = weight.shape
        assert weight_in_channels == in_channels, "weight's own in_channels must match x's own trailing dim"
        assert tuple(bias.shape) == (out_channels,), "bias must be [out_channels]"
        assert H % 2 == 0, f"H ({H}) must be even"
        assert W % 2 == 0, f"W ({W}) must be even"
        assert in_channels % 16 == 0, f"in_channels ({in_channels}) must be a multiple of 16"
        assert out_channels % 16 == 0, f"out_channels ({out_channels}) must be a multiple of 16"
        assert in_channels <= 64, f"in_channels ({in_channels}) must be at most 64"
        assert out_channels <= 1024, f"out_channels ({out_channels}) must be at most 1024"
        if bias.scalar_type != torch.float32:
            raise TypeError("bias must be a float32 buffer (reference field is Buffer[FLOAT32])")
        self.CIN, self.COUT, self.H, self.W = int(in_channels), int(out_channels), int(H), int(W)
        self.x_buf = data
        self.bias = bias
        self._desc = _conv.conv_desc(1, self.H, self.W, self.CIN, self.COUT, _lib.LAYOUT_HWC,
                                     _conv._dtype_code(data.as_tensor("torch"), "x"), _lib.LAYOUT_HWC,
                                     _lib.DTYPE_F32, False)
        _conv.validate(self._desc)
        self.weight_u = _conv.transform_weight(weight.as_tensor("torch"), _lib.WLAYOUT_RSCK)
        self._upstream = upstream
        super().__init__([hw, out_channels])

    def _forward(self) -> None:
        _conv.forward(self._desc, self.x_buf.as_tensor("torch"), self.weight_u, self.bias.as_tensor("torch"),
                      self._result_t)


class Downsample2xTensorOp(TensorOperation):
    """2x2 average pool, stride 2, over a flattened channels-last [H*W, C]
    input (H, W even); channels unchanged (reference: nn.py:1090-1107,
    shaders/tensors/downsample2x_tensor_op.h).  result [(H/2)(W/2), C] fp32;
    the four taps are summed left to right in fp32, then scaled by 0.25."""

    def __init__(self, x, H: int, W: int) -> None:
        data, shape, upstream = _as_op_input(x)
        assert len(shape) == 2, "Downsample2xTensorOp requires a 2D (H*W, C) input"
        hw, channels = shape
        assert hw == H * W, f"H*W ({H * W}) must match x's own row count ({hw})"
        assert H % 2 == 0 and W % 2 == 0, "Downsample2xTensorOp requires even H and W"
        self.x_buf = _op_float32(data, "x")
        self.W = W // 2  # output width (the reference's field)
        self._in_hw = (int(H), int(W))
        self._upstream = upstream
        super().__init__([(H // 2) * (W // 2), channels])

    def _forward(self) -> None:
        _tensor_ops.downsample2x(self.x_buf.as_tensor("torch"), *self._in_hw, self._result_t)


class Upsample2xTensorOp(TensorOperation):
    """Nearest-neighbour 2x upsample over a flattened channels-last [H*W, C]
    input; channels unchanged (reference: nn.py:1110-1125,
    shaders/tensors/upsample2x_tensor_op.h).  result [(2H)(2W), C] fp32."""

    def __init__(self, x, H: int, W: int) -> None:
        data, shape, upstream = _as_op_input(x)
        assert len(shape) == 2, "Upsample2xTensorOp requires a 2D (H*W, C) input"
        hw, channels = shape
        assert hw == H * W, f"H*W ({H * W}) must match x's own row count ({hw})"
        self.x_buf = _op_float32(data, "x")
        self.W = W * 2  # output width (the reference's field)
        self._in_hw = (int(H), int(W))
        self._upstream = upstream
        super().__init__([(H * 2) * (W * 2), channels])

    def _forward(self) -> None:
        _tensor_ops.upsample2x(self.x_buf.as_tensor("torch"), *self._in_hw, self._result_t)


class ConcatTensorOp(TensorOperation):
    """Channel concat of two ops or tensors with the same row count
    (reference: nn.py:1128-1150, shaders/tensors/concat_tensor_op.h); both
    channel counts must be multiples of 8.  result [rows, C1 + C2] fp32."""

    def __init__(self, g1, g2) -> None:
        data1, shape1, up1 = _as_op_input(g1)
        data2, shape2, up2 = _as_op_input(g2)
        assert len(shape1) == 2 and len(shape2) == 2, "ConcatTensorOp requires 2D (H*W, C) inputs"
        assert shape1[0] == shape2[0], "g1/g2 must share the same H*W leading dim"
        assert shape1[1] % 8 == 0, f"g1's own channels ({shape1[1]}) must be a multiple of 8"
        assert shape2[1] % 8 == 0, f"g2's own channels ({shape2[1]}) must be a multiple of 8"
        self.x1_buf = _op_float32(data1, "g1")
        self.x2_buf = _op_float32(data2, "g2")
        self.C1 = int(shape1[1])
        self._upstream = up1
        self._extra_upstreams = (up2,) if up2 is not None else ()
        super().__init__([shape1[0], shape1[1] + shape2[1]])

    def _forward(self) -> None:
        _tensor_ops.concat(self.x1_buf.as_tensor("torch"), self.x2_buf.as_tensor("torch"), self._result_t)


# ------------------------------------------------------- direct convolutions
class _Conv2DTensorOpBase(TensorOperation):
    """'same'-padded (zero border), stride-1 2-D convolution over a flattened
    channels-last x [H*W, in_channels] (a buffer or an upstream
    TensorOperation), weight [KH, KW, in_channels, out_channels], bias
    [out_channels]; result [H*W, out_channels] fp32.  The weight is read (and,
    for the fp16 variants, rounded) at every dispatch, so in-place updates of
    it are seen by evaluate().  One implicit-GEMM matrix-core kernel serves
    every variant (rdv_conv2d)."""

    _precision = _lib.PREC_F16

    def _bind(self, x, weight, bias, H: int, W: int, fixed_3x3: bool = False):
        name = type(self).__name__
        data, shape, upstream = _as_op_input(x)
        assert len(shape) == 2, f"{name} requires a 2D (H*W, in_channels) input"
        hw, in_channels = shape
        assert hw == H * W, f"H*W ({H * W}) must match x's own row count ({hw})"
        weight = weight if isinstance(weight, RDVObject) else wrap(weight)
        bias = bias if isinstance(bias, RDVObject) else wrap(bias)
        if fixed_3x3:
            assert tuple(weight.shape[:2]) == (3, 3), "weight must be [3, 3, in_channels, out_channels]"
        else:
            assert len(weight.shape) == 4, "weight must be [KH, KW, in_channels, out_channels]"
        kh, kw, weight_in_channels, out_channels = weight.shape
        assert weight_in_channels == in_channels, "weight's own in_channels must match x's own trailing dim"
        assert tuple(bias.shape) == (out_channels,), "bias must be [out_channels]"
        self.x_buf = _op_float32(data, "x")
        self.weight = _op_float32(weight, "weight")
        self.bias = _op_float32(bias, "bias")
        self._upstream = upstream
        self.KH, self.KW = int(kh), int(kw)
        self.CIN, self.COUT, self.H, self.W = int(in_channels), int(out_channels), int(H), int(W)
        return int(hw), int(in_channels), int(out_channels)

    def _finish(self) -> None:
        self._desc = _tensor_ops.conv2d_desc(self.H, self.W, self.CIN, self.COUT, self.KH, self.KW, self._precision,
                                             _lib.WLAYOUT_RSCK)
        _tensor_ops.conv2d_validate(self._desc, type(self).__name__)
        super().__init__([self.H * self.W, self.COUT])

    def _forward(self) -> None:
        _tensor_ops.conv2d(self._desc, self.x_buf.as_tensor("torch"), self.weight.as_tensor("torch"),
                           self.bias.as_tensor("torch"), self._result_t, type(self).__name__)


class Conv2DTensorOp(_Conv2DTensorOpBase):
    """fp32 throughout (reference: nn.py:414-470, shaders/tensors/conv2d_tensor_op.h):
    acc = bias; acc += x * w over the valid taps in (kh, kw) order and channels
    ascending.  H*W must be a multiple of 4, in_channels and out_channels
    multiples of 8."""

    _precision = _lib.PREC_F32

    def __init__(self, x, weight, bias, H: int, W: int) -> None:
        _, in_channels, out_channels = self._bind(x, weight, bias, H, W)
        assert in_channels % 8 == 0, f"in_channels ({in_channels}) must be a multiple of 8"
        assert out_channels % 8 == 0, f"out_channels ({out_channels}) must be a multiple of 8"
        self._finish()


class Conv2DTensorOpFast(_Conv2DTensorOpBase):
    """x and weight rounded to fp16, fp32 accumulation, fp32 bias added after
    (reference: nn.py:608-668, shaders/tensors/conv2d_tensor_op_fast.h).  H*W
    must be a multiple of 32, in_channels and out_channels multiples of 16."""

    _TILE_ROWS = 32
    _TILE_COLS = 16

    def __init__(self, x, weight, bias, H: int, W: int) -> None:
        _, in_channels, out_channels = self._bind(x, weight, bias, H, W)
        assert in_channels % 16 == 0, f"in_channels ({in_channels}) must be a multiple of 16"
        assert out_channels % 16 == 0, f"out_channels ({out_channels}) must be a multiple of 16"
        self._finish()


class Conv2DTensorOpSimple(_Conv2DTensorOpBase):
    """x and weight rounded to fp16, fp32 accumulation seeded with the bias
    (reference: nn.py:669-756, shaders/tensors/conv2d_tensor_op_simple.h).  H*W
    must be a multiple of 32, in_channels and out_channels multiples of 16."""

    _TILE_ROWS = 32
    _TILE_COLS = 16

    def __init__(self, x, weight, bias, H: int, W: int) -> None:
        hw, in_channels, out_channels = self._bind(x, weight, bias, H, W)
        assert hw % 32 == 0, f"H*W ({hw}) must be a multiple of 32"
        assert in_channels % 16 == 0, f"in_channels ({in_channels}) must be a multiple of 16"
        assert out_channels % 16 == 0, f"out_channels ({out_channels}) must be a multiple of 16"
        self._finish()


class Conv2DTensorOpSimple3x3(_Conv2DTensorOpBase):
    """3x3 kernel, padding 1; x and weight rounded to fp16, fp32 accumulation
    seeded with the bias (reference: nn.py:757-850,
    shaders/tensors/conv2d_tensor_op_simple3x3.h).  H*W must be a multiple of
    32, in_channels and out_channels multiples of 16.  SPT is the reference's
    subgroups-per-tile choice (_max_subgroups under its 48 KB budget); the HIP
    kernel's tiling does not depend on it."""

    _TILE_ROWS = 32
    _TILE_COLS = 16

    def __init__(self, x, weight, bias, H: int, W: int) -> None:
        hw, in_channels, out_channels = self._bind(x, weight, bias, H, W, fixed_3x3=True)
        assert hw % 32 == 0, f"H*W ({hw}) must be a multiple of 32"
        assert in_channels % 16 == 0, f"in_channels ({in_channels}) must be a multiple of 16"
        assert out_channels % 16 == 0, f"out_channels ({out_channels}) must be a multiple of 16"
        tap_k = 9 * in_channels
        self.SPT = _tensor_ops.max_subgroups(fixed_bytes=32 * tap_k * 2, per_subgroup_bytes=16 * tap_k * 2,
                                             divides=lambda s: out_channels % (16 * s) == 0)
        self._finish()


class Conv2DTensorOpWindow3x3(_Conv2DTensorOpBase):
    """3x3 kernel, padding 1; x and weight rounded to fp16, fp32 accumulation
    seeded with the bias (reference: nn.py:851-1000,
    shaders/tensors/conv2d_tensor_op_window3x3.h).  H and W must be multiples
    of 8, in_channels and out_channels multiples of 16, in_channels at most 64
    (the reference's shared-memory budget).  The reference pads x into a
    scratch buffer in a first dispatch; here the kernel zero-fills the border
    taps itself, so there is one dispatch and no scratch."""

    _WIN = 8
    _TILE_ROWS = 1
    _TILE_COLS = 16

    def __init__(self, x, weight, bias, H: int, W: int) -> None:
        _, in_channels, out_channels = self._bind(x, weight, bias, H, W, fixed_3x3=True)
        assert H % self._WIN == 0, f"H ({H}) must be a multiple of {self._WIN}"
        assert W % self._WIN == 0, f"W ({W}) must be a multiple of {self._WIN}"
        assert in_channels % 16 == 0, f"in_channels ({in_channels}) must be a multiple of 16"
        assert out_channels % 16 == 0, f"out_channels ({out_channels}) must be a multiple of 16"
        assert in_channels <= 64, f"in_channels ({in_channels}) must be at most 64 (see this op's own docstring)"
        fetch = self._WIN + 2
        shared_bytes = (fetch * fetch * in_channels + 16 * 9 * in_channels) * 2 + 64 * 16 * 2 + 64 * 16 * 4
        assert shared_bytes <= 49152, f"in_channels ({in_channels}) needs {shared_bytes} bytes of shared memory (48KB budget)"
        self._finish()
