"""Lowers a composed Map onto the fused MLP kernels (rdv_mlp_* in the C ABI).

A composition is accepted when its stages, in application order, are
  [FrequencyEncoding]? (Linear | LinearFast) [activation]? ( (Linear | LinearFast) [activation]? )*
which is what the reference's MapEvaluator runs for a chain of
`linear(...) >> relu >> ...` (src/rdv/maths/__init__.py:1451-1487,
src/rdv/shaders/maps/composite.h:8-12).  A Constant alone (maths:1659-1668) is
lowered as one layer with zero weights and the constant as its bias, which
the field kernels (extinctions, the renderer's field) evaluate exactly: every
product is 0 and the accumulator starts at the bias.  Anything else raises
NotImplementedError: this build has no general Map code generator.
"""
from __future__ import annotations

import ctypes as C
import math

import torch

from . import _lib
from .core import RDVObject, current_stream_handle, device, launch_scope, wrap
from .maths import Constant, Identity, Map
from .nn import FrequencyEncoding, _Activation, _LinearBase


class ChainPlan:
    __slots__ = ("desc", "layers", "signature", "in_features", "out_features", "ws_bytes", "arrays")

    def __init__(self, desc, layers, signature, in_features, out_features):
        self.desc = desc
        self.layers = layers
        self.signature = signature
        self.in_features = in_features
        self.out_features = out_features
        self.ws_bytes = None  # rdv_mlp_unpacked_workspace_bytes, once known
        self.arrays = None    # (pointer key, weight array, bias array) of the last call


class _ConstantLayer:
    """A Constant seen as a layer [OUT, in_width]: zero fp32 weights (one buffer
    kept on the Constant) and the constant's first OUT floats as the bias, read
    at every pack like any layer's bias."""

    def __init__(self, c: Constant, in_width: int) -> None:
        self.IN, self.OUT = int(in_width), int(c.OUT)
        self._precision = _lib.PREC_F16  # zero weights: the products are exact in any precision
        zero = c.__dict__.get("_rdv_zero_w")
        if zero is None or tuple(zero.shape) != (self.OUT, self.IN):
            zero = wrap(torch.zeros((self.OUT, self.IN), dtype=torch.float32, device=device()))
            c.__dict__["_rdv_zero_w"] = zero
        self.weight = zero
        self.bias = _ValuePtr(c._value_ptr())


class _ValuePtr:
    __slots__ = ("device_ptr",)

    def __init__(self, ptr: int) -> None:
        self.device_ptr = ptr


def _plan_constant(c: Constant, in_width: int) -> ChainPlan:
    lay = _ConstantLayer(c, in_width)
    d = _lib.MlpDesc()
    d.n_layers = 1
    d.in_features = in_width
    d.encoding = _lib.ENC_NONE
    d.enc_octaves = 0
    d.dims[0], d.dims[1] = in_width, lay.OUT
    d.act[0] = _lib.ACT_NONE
    d.prec[0] = lay._precision
    _lib.check(_lib.load().rdv_mlp_validate(C.byref(d)), "mlp")
    return ChainPlan(d, [lay], ("constant", in_width, lay.OUT), in_width, lay.OUT)


def plan_chain(m: Map, in_width: int) -> ChainPlan:
    """m's lowering for rows of in_width features.  A composition's structure
    never changes after it is built, so the plan is kept on m per input width
    (a Constant's is rebuilt: its value buffer may be converted per call)."""
    plans = m.__dict__.get("_rdv_plans")
    hit = plans.get(in_width) if plans is not None else None
    if hit is not None:
        return hit
    p = _plan_chain(m, in_width)
    if p.signature[0] != "constant":
        m.__dict__.setdefault("_rdv_plans", {})[in_width] = p
    return p


def _plan_chain(m: Map, in_width: int) -> ChainPlan:
    stages = [s for s in m.stages() if not isinstance(s, Identity)]
    if len(stages) == 1 and isinstance(stages[0], Constant):
        return _plan_constant(stages[0], in_width)
    enc, octaves, i, cur = _lib.ENC_NONE, 0, 0, in_width
    if stages and isinstance(stages[0], FrequencyEncoding):
        e = stages[0]
        if e.in_features != cur:
            raise TypeError(f"encoding expects {e.in_features} input features, x has {cur}")
        enc, octaves, cur, i = _lib.ENC_FREQ, e.octaves, e.OUT, 1
    enc_width = cur
    layers: list[_LinearBase] = []
    acts: list[int] = []
    for s in stages[i:]:
        if isinstance(s, _LinearBase):
            if s.IN != cur:
                raise TypeError(f"layer expects {s.IN} input features, the chain provides {cur}")
            layers.append(s)
            acts.append(_lib.ACT_NONE)
            cur = s.OUT
        elif isinstance(s, _Activation):
            if not layers:
                raise NotImplementedError("an activation before the first linear layer has no HIP lowering")
            if acts[-1] == _lib.ACT_NONE:
                acts[-1] = s._act
            elif acts[-1] == _lib.ACT_RELU and s._act == _lib.ACT_RELU:
                pass  # relu(relu(x)) == relu(x)
            else:
                raise NotImplementedError("two different activations in a row have no HIP lowering")
        elif isinstance(s, FrequencyEncoding):
            raise NotImplementedError("FrequencyEncoding is only supported as the first stage of a chain")
        else:
            raise NotImplementedError(f"{type(s).__name__} has no HIP lowering in this build")
    if not layers:
        raise NotImplementedError("a chain needs at least one Linear / LinearFast layer")
    if len(layers) > _lib.MLP_MAX_LAYERS:
        raise NotImplementedError(f"chains longer than {_lib.MLP_MAX_LAYERS} layers are not supported")
    d = _lib.MlpDesc()
    d.n_layers = len(layers)
    d.in_features = in_width
    d.encoding = enc
    d.enc_octaves = octaves
    d.dims[0] = enc_width
    for k, (lay, a) in enumerate(zip(layers, acts)):
        d.dims[k + 1] = lay.OUT
        d.act[k] = a
        d.prec[k] = lay._precision
    sig = (enc, octaves, in_width, tuple(d.dims[: d.n_layers + 1]), tuple(acts),
           tuple(l._precision for l in layers))
    _lib.check(_lib.load().rdv_mlp_validate(C.byref(d)), "mlp")
    return ChainPlan(d, layers, sig, in_width, cur)


def _param_arrays(p: ChainPlan):
    """The layers' weight and bias pointers as the C arrays the ABI takes,
    rebuilt only when a pointer changed."""
    key = tuple((l.weight.device_ptr, l.bias.device_ptr) for l in p.layers)
    if p.arrays is None or p.arrays[0] != key:
        p.arrays = (key, _lib.void_ptr_array([k[0] for k in key]), _lib.void_ptr_array([k[1] for k in key]))
    return p.arrays


def _packed_buffer(m: Map, p: ChainPlan) -> torch.Tensor:
    """m's packed-block buffer (256-byte aligned, cached per chain structure).
    Every call packs into it on the current stream; a call on another stream
    than the last first waits for that stream's work, so no kernel still
    reading the block sees it rewritten."""
    nbytes = int(_lib.load().rdv_mlp_packed_bytes(C.byref(p.desc)))
    if nbytes < 0:
        _lib.check(nbytes, "mlp")
    cached = m.__dict__.get("_rdv_packed")
    if cached is not None and cached[0] == p.signature:
        buf, last = cached[1], cached[2]
        cur = torch.cuda.current_stream()
        if last is not None and last != cur:
            cur.wait_stream(last)
        m.__dict__["_rdv_packed"] = (p.signature, buf, cur)
        return buf
    raw = torch.empty(nbytes + 256, dtype=torch.uint8, device=device())
    off = (-raw.data_ptr()) % 256
    buf = raw[off: off + nbytes]
    m.__dict__["_rdv_packed"] = (p.signature, buf, torch.cuda.current_stream())
    return buf


def packed_params(m: Map, p: ChainPlan) -> torch.Tensor:
    """Packed parameter block of `m`, re-packed from the layers' fp32 weight and
    bias buffers at every call (one launch, stream-ordered before the launch
    that reads it).  The reference reads weights through pointers at every
    dispatch, so any update of a weight buffer -- in place, through `.data`,
    through another alias or from outside torch -- is seen by the next
    evaluation.  Only the packed buffer itself is cached, so steady-state calls
    allocate nothing."""
    buf = _packed_buffer(m, p)
    _, ws, bs = _param_arrays(p)
    _lib.check(_lib.load().rdv_mlp_pack(C.byref(p.desc), ws, bs, C.c_void_p(buf.data_ptr()),
                                        C.c_void_p(current_stream_handle())), "mlp pack")
    return buf


_OUTPUT_CACHE: dict = {}


def _cached_output(sig, shape) -> RDVObject:
    """One output buffer per chain structure, reallocated only when the row shape
    changes (reference: Map.__call__'s per-class evaluator cache)."""
    hit = _OUTPUT_CACHE.get(sig)
    if hit is not None and hit[0] == shape:
        return hit[1]
    out = RDVObject(torch.empty(shape, dtype=torch.float32, device=device()))
    _OUTPUT_CACHE[sig] = (shape, out)
    return out


def evaluate_map(m: Map, x) -> RDVObject:
    x = wrap(x)
    if x.scalar_type != torch.float32:
        raise TypeError(f"Map input must be float32, got {x.scalar_type}")
    if len(x.shape) < 1:
        raise AssertionError("Map input needs a trailing feature dimension")
    p = plan_chain(m, int(x.shape[-1]))
    out = _cached_output(p.signature, (*x.shape[:-1], p.out_features))
    with launch_scope():
        _launch(m, p, x.device_ptr, out.device_ptr, math.prod(x.shape[:-1]))
    return out


def _launch(m: Map, p: ChainPlan, x_ptr: int, y_ptr: int, rows: int) -> None:
    """One rdv_mlp_forward_unpacked call: the layers' parameters are read at
    this call (a chain with a compile-time kernel converts them in the kernel;
    any other is packed into m's cached buffer first, in the same call)."""
    lib = _lib.load()
    if p.ws_bytes is None:
        nb = int(lib.rdv_mlp_unpacked_workspace_bytes(C.byref(p.desc)))
        if nb < 0:
            _lib.check(nb, "mlp")
        p.ws_bytes = nb
    _, ws, bs = _param_arrays(p)
    wsp = _packed_buffer(m, p).data_ptr() if p.ws_bytes else None
    _lib.check(lib.rdv_mlp_forward_unpacked(C.byref(p.desc), ws, bs, C.c_void_p(x_ptr), C.c_void_p(y_ptr),
                                            C.c_int64(rows), C.c_void_p(wsp), C.c_int64(p.ws_bytes),
                                            C.c_void_p(current_stream_handle())), "mlp forward")


def launch_map_rows(m: Map, x_ptr: int, y_ptr: int, rows: int) -> None:
    """m over `rows` rows of fp32 x at x_ptr into fp32 y at y_ptr (device
    pointers; m's input width must be known).  What MapEvaluator runs."""
    rows_fn = getattr(m, "_launch_rows", None)
    if rows_fn is not None:
        rows_fn(x_ptr, y_ptr, rows)
        return
    if m.IN is None:
        raise RuntimeError("Generic arguments could not be deduced from input data. You must explicitly cast.")
    _launch(m, plan_chain(m, int(m.IN)), x_ptr, y_ptr, rows)
