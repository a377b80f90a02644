"""Materialised grids and grid-to-grid operations of the rdv API, and the
staged evaluation of any grid graph.

  TensorGrid, barrier          reference: src/rdv/maths/__init__.py:487-531, 1613-1655
  Conv2dGrid / conv2d          src/rdv/domain/nn.py:122-188, shaders/grids/conv2d.h
  Conv2D / conv2d_o            nn.py:191-254, shaders/grids/conv2d_per_output.h
  Downsample2x, Upsample2x     nn.py:269-301, shaders/grids/{downsample2x,upsample2x}.h
  Sensor (any grid, any map)   maths:252-271, shaders/grids/sensor.h

The reference stitches a grid graph into one generated shader per root type
(_core.py:2514-2645) and evaluates every node inside every thread.  Here a
graph is evaluated node by node, each node one kernel over the whole grid
into an HBM-resident [*shape, OUT] buffer that the next node reads: a
convolution reads its input image once per tap from L2 instead of
re-evaluating the producer per tap, and a map runs on the matrix cores over
all rows at once.  The hot patterns keep their fused kernels (a camera
grid into EmissionAbsorption or RaymarchingTransmittance is one kernel,
_render.py).  Each node keeps its own output buffer and reuses it while the
shape is unchanged; one top-level evaluation computes each node once.
"""
from __future__ import annotations

import math

import torch

from . import _lib, _tensor_ops
from .core import RDVObject, device, wrap
from .maths import Grid, Map, Sensor
from .types import Generic, Generics


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.float32 and t.is_contiguous() else t.to(torch.float32).contiguous()


class _GridNode(Grid):
    """A grid whose values come from a kernel over its inputs' values."""

    def _out(self, shape) -> RDVObject:
        shape = tuple(int(s) for s in shape)
        cached = self.__dict__.get("_rdv_out")
        if cached is None or tuple(cached.shape) != shape:
            cached = RDVObject(torch.empty(shape, dtype=torch.float32, device=device()))
            self.__dict__["_rdv_out"] = cached
        return cached

    def _values(self, ctx: dict) -> RDVObject:  # launches this node's kernel
        raise NotImplementedError


def grid_values(g: Grid, ctx: dict) -> RDVObject:
    """g's values [*shape, OUT] (fp32, on the GPU), each node once per ctx."""
    key = id(g)
    hit = ctx.get(key)
    if hit is not None:
        return hit[1]
    from . import _render
    if isinstance(g, _GridNode):
        v = g._values(ctx)
    elif isinstance(g, Sensor):
        v = _sensor_values(g, ctx)
    else:
        v = _render.evaluate_grid(g)
    ctx[key] = (g, v)
    return v


def _sensor_values(s: Sensor, ctx: dict) -> RDVObject:
    """map(grid(idx)) for every cell: the grid's values, then the map over all
    of its rows (reference: Sensor, maths:252-271)."""
    from . import _chain, _render
    from .rendering import Cameras, EmissionAbsorption
    if isinstance(s.grid, Cameras):
        return _render.evaluate_grid(s)
    gv = grid_values(s.grid, ctx)
    rows = math.prod(s.grid.shape)
    out = s.__dict__.get("_rdv_out")
    shape = (*s.grid.shape, int(s.map.OUT))
    if out is None or tuple(out.shape) != shape:
        out = RDVObject(torch.empty(shape, dtype=torch.float32, device=device()))
        s.__dict__["_rdv_out"] = out
    m = s.map
    if isinstance(m, EmissionAbsorption):
        _render.render_ea_rays(m, gv.device_ptr, out.device_ptr, rows)
    else:
        _chain.launch_map_rows(m, gv.device_ptr, out.device_ptr, rows)
    return out


# ------------------------------------------------------------ tensor grids


class TensorGrid(_GridNode):
    """A tensor [*shape, OUT] seen as a grid over its leading dimensions
    (reference: maths:487-505).  Cell values are read from the tensor."""

    def __init__(self, data) -> None:
        if not isinstance(data, RDVObject):
            data = wrap(data)
        shape = list(data.shape)
        self.IN = len(shape) - 1
        self.OUT = int(shape[-1])
        super().__init__(shape[:-1])
        self.ptr = data

    def _values(self, ctx: dict) -> RDVObject:
        t = self.ptr.as_tensor("torch")
        if t.dtype != torch.float32 or not t.is_contiguous():
            return wrap(_f32(t))
        return self.ptr


class TensorGridBarrier(TensorGrid):
    """`grid >> barrier`: a tensor grid holding `grid`'s values, recomputed
    from `grid` each time an evaluation reads it (reference: maths:508-531)."""

    def __init__(self, grid, **kwargs) -> None:
        assert not kwargs, f"TensorGridBarrier takes no extra arguments, got {kwargs!r}"
        if grid.OUT is None:
            raise RuntimeError("Generic arguments could not be deduced: the grid's OUT is unknown")
        _GridNode.__init__(self, list(grid.shape))
        self.IN = grid.IN
        self.OUT = int(grid.OUT)
        self._source = grid
        self.ptr = None  # allocated on first evaluation

    def _values(self, ctx: dict) -> RDVObject:
        v = grid_values(self._source, ctx)
        if self.ptr is None:
            self.ptr = self._out((*self.shape, self.OUT))
        if v.device_ptr != self.ptr.device_ptr:
            self.ptr.as_tensor("torch").copy_(v.as_tensor("torch").reshape(self.ptr.shape))
        return self.ptr


TensorGrid.__barrier_type__ = TensorGridBarrier


class _BarrierDeclaration:
    """`grid >> barrier` materialises any grid into a TensorGrid (reference:
    maths:1613-1655); barrier[TensorGrid] names the target type."""

    def __init__(self, target=None, kwargs=None) -> None:
        self._target = target
        self._kwargs = kwargs

    def __call__(self, **kwargs):
        assert self._kwargs is None, "Arguments of barrier can not be set twice"
        return _BarrierDeclaration(self._target, kwargs)

    def __getitem__(self, item):
        assert isinstance(item, type) and hasattr(item, "__barrier_type__")
        assert self._target is None, "Result type of a barrier can not be set twice"
        return _BarrierDeclaration(item, self._kwargs)

    def create_barrier(self, grid):
        target = self._target or TensorGrid
        return target.__barrier_type__(grid, **(self._kwargs or {}))

    def __rrshift__(self, other):
        if not isinstance(other, Grid):
            return NotImplemented
        return self.create_barrier(other)


barrier = _BarrierDeclaration()


# -------------------------------------------------------- grid convolutions


def _as_rdv(t) -> RDVObject:
    return t if isinstance(t, RDVObject) else wrap(t)


class Conv2dGrid(_GridNode, Generic[Generics.G, Generics.KH, Generics.KW, Generics.CIN]):
    """'same'-padded (zero border), stride-1 2-D convolution over a grid g of
    shape (H, W) and OUT = in_channels; weight [out_channels, in_channels, KH,
    KW] (PyTorch nn.Conv2d layout), bias [out_channels]; OUT = out_channels
    (reference: nn.py:122-166, shaders/grids/conv2d.h: fp32, accumulator
    seeded with the bias, taps in (kh, kw) order, channels ascending).  Built
    by `g >> conv2d(weight, bias)`."""

    def __init__(self, g, weight, bias) -> None:
        weight = _as_rdv(weight)
        bias = _as_rdv(bias)
        assert len(weight.shape) == 4, "weight must be [out_channels, in_channels, KH, KW]"
        out_channels, in_channels, kh, kw = weight.shape
        assert tuple(bias.shape) == (out_channels,), "bias must be [out_channels]"
        assert g.OUT == in_channels, "g's own OUT must match weight's in_channels"
        assert len(g.shape) == 2, "g must be a 2D (H, W) grid"
        self.match(Generics.KH, int(kh))
        self.match(Generics.KW, int(kw))
        self.match(Generics.CIN, int(in_channels))
        super().__init__(list(g.shape))
        self.IN = g.IN
        self.OUT = int(out_channels)
        self.g = g
        self.weight = weight
        self.bias = bias

    def _values(self, ctx: dict) -> RDVObject:
        H, W = self.shape
        x = grid_values(self.g, ctx)
        out = self._out((H, W, self.OUT))
        cout, cin, kh, kw = self.weight.shape
        d = _tensor_ops.conv2d_desc(H, W, cin, cout, kh, kw, _lib.PREC_F32, _lib.WLAYOUT_KCRS)
        _tensor_ops.conv2d(d, x.as_tensor("torch").reshape(H * W, cin), _f32(self.weight.as_tensor("torch")),
                           _f32(self.bias.as_tensor("torch")), out.as_tensor("torch").reshape(H * W, cout),
                           "Conv2dGrid")
        return out


class _Conv2dDeclaration:
    def __init__(self, weight, bias) -> None:
        self.weight = weight
        self.bias = bias

    def __rrshift__(self, other):
        if not isinstance(other, Grid):
            return NotImplemented
        return Conv2dGrid(other, self.weight, self.bias)


def conv2d(weight, bias) -> _Conv2dDeclaration:
    """`g >> conv2d(weight, bias)` builds Conv2dGrid(g, weight, bias)."""
    return _Conv2dDeclaration(weight, bias)


class Conv2D(_GridNode, Generic[Generics.G, Generics.KH, Generics.KW, Generics.CIN, Generics.COUT]):
    """The same convolution with one cell per (h, w, out channel): shape
    (H, W, out_channels, 1), OUT = 1; weight [KH, KW, in_channels,
    out_channels] (channels-last), bias [out_channels] (reference:
    nn.py:191-254, shaders/grids/conv2d_per_output.h).  Built by
    `g >> conv2d_o(weight, bias)`."""

    def __init__(self, g, weight, bias) -> None:
        weight = _as_rdv(weight)
        bias = _as_rdv(bias)
        assert len(weight.shape) == 4, "weight must be [KH, KW, in_channels, out_channels]"
        kh, kw, in_channels, out_channels = weight.shape
        assert tuple(bias.shape) == (out_channels,), "bias must be [out_channels]"
        assert g.OUT == in_channels, "g's own OUT must match weight's in_channels"
        assert len(g.shape) == 2, "g must be a 2D (H, W) grid"
        H, W = g.shape
        self.match(Generics.KH, int(kh))
        self.match(Generics.KW, int(kw))
        self.match(Generics.CIN, int(in_channels))
        self.match(Generics.COUT, int(out_channels))
        super().__init__([H, W, int(out_channels), 1])
        self.IN = 4
        self.OUT = 1
        self.g = g
        self.weight = weight
        self.bias = bias

    def _values(self, ctx: dict) -> RDVObject:
        H, W, cout, _ = self.shape
        x = grid_values(self.g, ctx)
        out = self._out((H, W, cout, 1))
        kh, kw, cin, _ = self.weight.shape
        d = _tensor_ops.conv2d_desc(H, W, cin, cout, kh, kw, _lib.PREC_F32, _lib.WLAYOUT_RSCK)
        _tensor_ops.conv2d(d, x.as_tensor("torch").reshape(H * W, cin), _f32(self.weight.as_tensor("torch")),
                           _f32(self.bias.as_tensor("torch")), out.as_tensor("torch").reshape(H * W, cout), "Conv2D")
        return out


class _Conv2DDeclaration:
    def __init__(self, weight, bias) -> None:
        self.weight = weight
        self.bias = bias

    def __rrshift__(self, other):
        if not isinstance(other, Grid):
            return NotImplemented
        return Conv2D(other, self.weight, self.bias)


def conv2d_o(weight, bias) -> _Conv2DDeclaration:
    """`g >> conv2d_o(weight, bias)` builds Conv2D(g, weight, bias)."""
    return _Conv2DDeclaration(weight, bias)


class Downsample2x(_GridNode, Generic[Generics.G]):
    """2x2 average pool, stride 2, over a 2-D grid (H, W even); OUT unchanged
    (reference: nn.py:269-285, shaders/grids/downsample2x.h:
    0.25 * (v00 + v01 + v10 + v11), summed left to right in fp32)."""

    def __init__(self, g) -> None:
        assert len(g.shape) == 2, "Downsample2x requires a 2D (H, W) grid"
        H, W = g.shape
        assert H % 2 == 0 and W % 2 == 0, "Downsample2x requires even H and W"
        super().__init__([H // 2, W // 2])
        self.IN = 2
        self.OUT = g.OUT
        self.g = g

    def _values(self, ctx: dict) -> RDVObject:
        H, W = self.g.shape
        x = grid_values(self.g, ctx)
        out = self._out((H // 2, W // 2, self.OUT))
        _tensor_ops.downsample2x(x.as_tensor("torch").reshape(H * W, self.OUT), H, W,
                                 out.as_tensor("torch").reshape(-1, self.OUT))
        return out


class Upsample2x(_GridNode, Generic[Generics.G]):
    """Nearest-neighbour 2x upsample of a 2-D grid; OUT unchanged (reference:
    nn.py:288-301, shaders/grids/upsample2x.h)."""

    def __init__(self, g) -> None:
        assert len(g.shape) == 2, "Upsample2x requires a 2D (H, W) grid"
        H, W = g.shape
        super().__init__([H * 2, W * 2])
        self.IN = 2
        self.OUT = g.OUT
        self.g = g

    def _values(self, ctx: dict) -> RDVObject:
        H, W = self.g.shape
        x = grid_values(self.g, ctx)
        out = self._out((2 * H, 2 * W, self.OUT))
        _tensor_ops.upsample2x(x.as_tensor("torch").reshape(H * W, self.OUT), H, W,
                               out.as_tensor("torch").reshape(-1, self.OUT))
        return out


class MajorantGrid(_GridNode, Generic[Generics.G]):
    """`grid` at a new (typically coarser) `shape`: each cell holds the
    channel-wise maximum over every cell of `grid` that a sampler with the same
    aligned / linear convention could read from anywhere inside it (a linear
    sampler reaches one cell past the naive range); the bound that voxel
    majorant fields need (reference: maths:534-569, shaders/grids/majorant_grid.h).
    Grids of 1 to 4 dimensions."""

    def __init__(self, grid, shape: list[int], aligned: bool = False, linear: bool = True) -> None:
        assert len(shape) == len(grid.shape), "MajorantGrid keeps the grid's dimension count"
        assert 1 <= len(shape) <= 4, "MajorantGrid supports 1 to 4 dimensions"
        super().__init__(list(shape))
        self.IN = grid.IN
        self.OUT = grid.OUT
        self.grid = grid
        self.aligned = 1 if aligned else 0
        self.linear = 1 if linear else 0

    def _values(self, ctx: dict) -> RDVObject:
        from . import _render
        fine = grid_values(self.grid, ctx).as_tensor("torch")
        fine = _f32(fine)
        out = self._out((*self.shape, self.OUT))
        _render.majorant_grid(fine, self.grid.shape, self.shape, int(self.OUT), bool(self.aligned),
                              bool(self.linear), out.as_tensor("torch"))
        return out
