"""Map / Grid / TensorOperation families of the rdv API, for the hot path.

Reference: src/rdv/maths/__init__.py.  A Map is a per-row function
[..., IN] -> [..., OUT]; `a >> b` composes (b after a) into a Composite
(maths:1489-1498, 1700-1728); calling a Map evaluates it over every row of its
input (maths:1451-1487).  The reference lowers a composition to one GLSL
shader; here a composition is pattern-matched onto the fused HIP kernels
(see _chain.py), and anything that does not match raises NotImplementedError.
"""
from __future__ import annotations

import math as _math

from .core import RDVObject, wrap
from .types import IN as _IN, OUT as _OUT
from .types import Component, DeferredLibrary, Generic, Generics, Main, generic_value


class Map(Component, Generic[_IN, _OUT]):
    """Base of every per-row map (reference: maths:1436).  IN / OUT are None
    while generic; Map[IN, OUT] is the specialisation, and isinstance(m,
    Map[3, 1]) holds for any map of those widths."""

    IN: int | None = None
    OUT: int | None = None

    def cast(self, target):
        """This map as a `target` (e.g. Map[3, 1]): its known widths must
        agree (reference: Node.cast, _core.py:1778-1814, as Map.__rshift__
        and ExtinctionTrait use it).  Maps here carry their widths per
        instance, so a compatible map is returned as it is."""
        origin = target.__dict__.get("__rdv_origin__", target) if isinstance(target, type) else None
        if origin is None or not isinstance(self, origin):
            raise TypeError(f"cannot cast {type(self).__name__} to {getattr(target, '__name__', target)}")
        for k, v in getattr(target, "__generics__", {}).items():
            cur = generic_value(self, k)
            if v is not None and cur is not None and cur != v:
                raise TypeError(f"cannot cast {type(self).__name__}: {k} is {cur}, {target.__name__} needs {v}")
        return self

    # ---------------------------------------------------------- composition
    def __rshift__(self, m: "Map") -> "Map":
        """self, then m (reference: Map.__rshift__, maths:1489-1498)."""
        if not isinstance(m, Map):
            return NotImplemented
        if isinstance(m, Identity):
            return self
        if isinstance(self, Identity):
            return m
        _check_link(self, m)
        return Composite(m, self)

    def __lshift__(self, m: "Map") -> "Map":
        """m, then self (reference: Map.__lshift__)."""
        if not isinstance(m, Map):
            return NotImplemented
        return m >> self

    def stages(self) -> list["Map"]:
        """Primitive maps in application order."""
        return [self]

    def __call__(self, x, **kwargs):
        """Evaluates the map over every row of x; returns a cached output object
        (same buffer when the same structure is called with the same row shape,
        as the reference's per-class evaluator cache does, maths:1466-1476).
        Keyword arguments bind deferred names for the duration of the call
        (reference: DeferredLibrary.bind around the dispatch, maths:1481-1486)."""
        if kwargs:
            DeferredLibrary.bind(**kwargs)
        try:
            ev = getattr(self, "_evaluate_rows", None)
            if ev is not None:  # maps with a kernel of their own (rendering nodes)
                return ev(x)
            from . import _chain
            return _chain.evaluate_map(self, x)
        finally:
            if kwargs:
                DeferredLibrary.unbind(**kwargs)


def _check_link(g: Map, f: Map) -> None:
    """g's OUT must equal f's IN once both are known (reference: Composite.__init__
    asserts it; a generic cast that cannot bind raises TypeError)."""
    go, fi = g.OUT, f.IN
    if go is not None and fi is not None and go != fi:
        raise TypeError(f"cannot compose: output width {go} does not match input width {fi}")


class Identity(Map):
    """f(x) = x (reference: maths:1671-1684)."""


X = Identity()


class Constant(Map):
    """f(x) = data for every row, whatever the input width (reference:
    maths:1659-1668, shaders/maps/constant.h).  data: [..., OUT]; the constant
    is the first OUT floats of the buffer (its first row), which is what the
    reference's shader copies; further rows are ignored."""

    def __init__(self, data) -> None:
        if not isinstance(data, RDVObject):
            data = wrap(data)
        self.OUT = int(data.shape[-1])
        self.buf_ = data

    def _value_ptr(self) -> int:
        import torch
        t = self.buf_.as_tensor("torch")
        if t.dtype != torch.float32 or not t.is_contiguous():
            t = t.to(torch.float32).contiguous()
            self.__dict__["_rdv_value"] = t  # keep the converted copy alive
        return t.data_ptr()

    def _launch_rows(self, x_ptr: int, y_ptr: int, rows: int) -> None:
        import ctypes as C
        from . import _lib
        from .core import current_stream_handle
        _lib.check(_lib.load().rdv_broadcast_rows(C.c_void_p(self._value_ptr()), C.c_int32(self.OUT),
                                                  C.c_int64(rows), C.c_void_p(y_ptr),
                                                  C.c_void_p(current_stream_handle())), "Constant")

    def _evaluate_rows(self, x) -> RDVObject:
        import torch
        from .core import device, launch_scope
        x = wrap(x)
        rows = _math.prod(x.shape[:-1]) if len(x.shape) >= 1 else 1
        hit = self.__dict__.get("_rdv_out")
        shape = (*x.shape[:-1], self.OUT)
        if hit is None or tuple(hit.shape) != shape:
            hit = RDVObject(torch.empty(shape, dtype=torch.float32, device=device()))
            self.__dict__["_rdv_out"] = hit
        with launch_scope():
            self._launch_rows(x.device_ptr, hit.device_ptr, rows)
        return hit


class Composite(Map):
    """f(g(x)) (reference: maths:1700-1728)."""

    def __init__(self, f: Map, g: Map) -> None:
        self.f = f
        self.g = g
        st = self.stages()
        self.IN = _infer_in(st)
        self.OUT = _infer_out(st)

    def stages(self) -> list[Map]:
        return self.g.stages() + self.f.stages()


def _infer_in(stages: list[Map]) -> int | None:
    for s in stages:
        if s.IN is not None:
            return s.IN
        if s.OUT is not None and not getattr(s, "_shape_preserving", False):
            return None
    return None


def _infer_out(stages: list[Map]) -> int | None:
    for s in reversed(stages):
        if s.OUT is not None:
            return s.OUT
        if not getattr(s, "_shape_preserving", False):
            return None
    return None


# ================================================================= GRIDS


class Grid(Component, Generic[_IN, _OUT]):
    """Index space [0..shape[i]) -> float vectors of width OUT (reference: maths:42-225).

    Calling a grid with no arguments evaluates every cell in row-major order
    into a [*shape, OUT] tensor (maths:77-103)."""

    IN: int | None = None
    OUT: int | None = None

    def __init__(self, shape: list[int]) -> None:
        self._shape = list(shape)
        self.shape = list(shape)

    def cast(self, target):
        """This grid as a `target` (e.g. Grid[3, 1]): its known IN / OUT must
        agree (reference: Node.cast, _core.py:1778-1814; the rules of Map.cast)."""
        return Map.cast(self, target)

    def __rshift__(self, m):
        if isinstance(m, Identity):
            return self
        if isinstance(m, Map):
            return Sensor(self, m)
        return NotImplemented

    def __call__(self, *args, **kwargs):
        """With no argument, every cell in row-major order into a cached
        [*shape, OUT] buffer (maths:77-103).  With one argument, a batch of
        index vectors [..., IN] (integers; the grid's IN-sized index in the
        last dimension): the grid at those indices only, into a cached
        [..., OUT] buffer, one thread per index vector (maths:104-119,
        BatchGridEvaluator).  Keyword arguments bind deferred names for the
        call."""
        assert len(args) <= 1, "Grid.__call__ takes at most one batch of indices"
        if kwargs:
            DeferredLibrary.bind(**kwargs)
        try:
            from . import _render
            if args:
                return _render.evaluate_grid_batch(self, args[0])
            return _render.evaluate_grid(self)
        finally:
            if kwargs:
                DeferredLibrary.unbind(**kwargs)


class Sensor(Grid):
    """map(grid(idx)) for every cell (reference: maths:252-271)."""

    def __init__(self, grid: Grid, map: Map) -> None:
        if map.IN is not None and grid.OUT is not None and map.IN != grid.OUT:
            raise TypeError(f"cannot compose: grid output width {grid.OUT} does not match map input {map.IN}")
        super().__init__(grid.shape)
        self.grid = grid
        self.map = map
        self.IN = grid.IN
        self.OUT = map.OUT


# ======================================================== TENSOR OPERATIONS


class TensorOperation(Component):
    """Self-materialising 2-D op, dispatched eagerly at construction
    (reference: maths:1251-1380).  Subclasses set up their inputs and call
    super().__init__(shape); `result` then holds the [rows, cols] fp32 output.
    rows and cols must be multiples of the class's _TILE_ROWS / _TILE_COLS
    (maths:1335-1337)."""

    _upstream = None
    _extra_upstreams = ()
    _TILE_ROWS = 4  # BLOCK_ROWS (maths:945)
    _TILE_COLS = 8  # BLOCK_CHANNELS (maths:946)

    def __init__(self, shape: list[int]) -> None:
        import torch
        from .core import device
        cls = type(self)
        assert len(shape) == 2, "TensorOperation only supports 2D (rows, channels) shapes"
        assert shape[0] % cls._TILE_ROWS == 0, f"rows ({shape[0]}) must be a multiple of {cls._TILE_ROWS}"
        assert shape[1] % cls._TILE_COLS == 0, f"channels ({shape[1]}) must be a multiple of {cls._TILE_COLS}"
        self._shape = list(shape)
        self.shape = list(shape)
        self._result_t = torch.empty(self._shape, dtype=torch.float32, device=device())
        self.result = RDVObject(self._result_t)
        self.evaluate()

    def _forward(self) -> None:  # launches this op's kernel into self._result_t
        raise NotImplementedError

    def as_type(self, backend: str):
        """This op's result in `backend` ('torch' view or 'numpy' copy)."""
        return self.result.as_tensor(backend).reshape(self._shape)

    def evaluate(self) -> None:
        """Re-dispatches this op over its own result buffer (maths:1360-1366)."""
        from .core import launch_scope
        with launch_scope():
            self._forward()

    def evaluate_chain(self) -> None:
        """Re-dispatches this op and every upstream op, in dependency order
        (maths:1368-1379)."""
        ops: list[TensorOperation] = []
        _collect_tensor_ops(self, set(), ops)
        for op in ops:
            op.evaluate()


def _as_op_input(x):
    """(buffer, shape, upstream op or None) of an op input (maths:1402-1415)."""
    if isinstance(x, TensorOperation):
        return x.result, list(x._shape), x
    data = wrap(x)
    return data, list(data.shape), None


def _collect_tensor_ops(node, seen_ids, out) -> None:
    """Postorder walk of upstream ops (maths:1418-1430)."""
    if id(node) in seen_ids:
        return
    if node._upstream is not None:
        _collect_tensor_ops(node._upstream, seen_ids, out)
    for up in node._extra_upstreams:
        _collect_tensor_ops(up, seen_ids, out)
    seen_ids.add(id(node))
    out.append(node)


pi = _math.pi
e = _math.e


# ============================================================== EVALUATORS


def _pointer_of(v) -> int:
    if isinstance(v, RDVObject):
        return v.device_ptr
    if hasattr(v, "data_ptr"):
        return int(v.data_ptr())
    return int(v)


class MapEvaluator(Main):
    """Evaluates `map` over rows: input [rows, IN] fp32 at `input`, output
    [rows, OUT] fp32 at `output` (RDVObjects or raw device pointers);
    dispatch(evaluator, rows) runs it (reference: maths:1569-1610)."""

    def __init__(self, map, input, output) -> None:
        self.map = map
        self.input_ptr = _pointer_of(input)
        self.output_ptr = _pointer_of(output)

    def set_direct(self, map, input_ptr: int, output_ptr: int) -> None:
        self.map, self.input_ptr, self.output_ptr = map, int(input_ptr), int(output_ptr)

    def _dispatch(self, threads: int) -> None:
        from . import _chain
        _chain.launch_map_rows(self.map, self.input_ptr, self.output_ptr, threads)


class GridEvaluator(Main):
    """Evaluates every cell of `grid` into `output` ([*shape, OUT] fp32, an
    RDVObject or a torch tensor); dispatch(evaluator, cells) runs it
    (reference: maths:785-812)."""

    def __init__(self, grid, output) -> None:
        self.g = grid
        self.output = output

    def set_direct(self, g, output) -> None:
        self.g, self.output = g, output

    def _dispatch(self, threads: int) -> None:
        from . import _render
        import math as _m
        want = _m.prod(self.g.shape)
        if threads != want:
            raise AssertionError(f"GridEvaluator dispatches one thread per cell ({want}), got {threads}")
        out = self.output if isinstance(self.output, RDVObject) else wrap(self.output)
        _render.evaluate_grid(self.g, out=out)


class BatchGridEvaluator(Main):
    """Evaluates `grid` at a batch of integer index vectors `input` ([rows, IN],
    int32 or another integer type; an RDVObject or a torch tensor) into
    `output` ([rows, OUT] fp32), one thread per index vector; dispatch(evaluator,
    rows) runs it (reference: maths:815-844, shaders/grids/batch_grid_evaluator.h)."""

    def __init__(self, grid, input, output) -> None:
        self.g = grid
        self.input = input
        self.output = output

    def set_direct(self, g, input, output) -> None:
        self.g, self.input, self.output = g, input, output

    def _dispatch(self, threads: int) -> None:
        from . import _render
        from .core import launch_scope
        idx, _, rows = _render._batch_indices(self.g, self.input)
        if threads != rows:
            raise AssertionError(f"BatchGridEvaluator dispatches one thread per index vector ({rows}), got {threads}")
        out = self.output if isinstance(self.output, RDVObject) else wrap(self.output)
        if tuple(out.shape)[-1:] != (int(self.g.OUT),) or _math.prod(out.shape) != rows * int(self.g.OUT):
            raise AssertionError(f"output must hold {rows} rows of {int(self.g.OUT)} floats, got {tuple(out.shape)}")
        with launch_scope():
            _render._batch_values(self.g, idx, rows, out.device_ptr, {})


class TensorOpEvaluator(Main):
    """Re-runs a TensorOperation's kernel over its own result buffer
    (reference: maths:1382-1399)."""

    def __init__(self, op) -> None:
        self.op = op

    def _dispatch(self, threads: int) -> None:
        self.op._forward()
