"""Node classes, generics, value types and deferred pointers of the rdv API.

Restates, for this build, the type system the reference keeps in
src/rdv/core/_core.py and src/rdv/core/_common.py, minus the GLSL code
generation it exists to drive there:

  GenericParam / Generics / Generic    _core.py:385-721
      Generics.T is a named parameter; `class A(Struct, Generic[T])` declares
      it; A[int], A[T: int] (or A[Generics.T: int]) bind it and give a cached
      specialisation whose name follows the declaration order.
  __aliases__                          _core.py:1391-1464 (alias rules)
      names fixed per class (resolved afresh for each specialisation), never
      redefined by a subclass, never a generic, never a binding target.
  Node.match / Node.cast                _core.py:1735-1814
      match() binds a still-open parameter from constructor data; cast()
      rebinds an instance to a specialisation of one of its base classes by
      replaying its constructor.
  _dependency_order                    _core.py:1578-1614
      post-order topological sort over __requires__.
  Type, Single, Array, Pointer, Buffer, FixArray,
  Deferred / deferreds / DeferredLibrary   _common.py:100-311
      field types; a Deferred names a buffer that is bound per call
      (`m(x, name=tensor)`, `grid(name=tensor)` or `with deferreds(...)`).
  vec2..vec4, ivec*, uvec*, bvec*, mat2..mat4, mat3x4, mat4x3
      GLSL value types (column-major matrices), as vulky provides them.

The reference generates shader structs from these declarations; here they
only carry the semantics callers observe (names, binding rules, errors), and
the compute kernels take their shapes from the descriptors built in
_chain.py / _render.py.
"""
from __future__ import annotations

import enum as _enum
import itertools as _itertools
import threading as _threading

# ================================================================ generics


class GenericParam:
    """A named generic parameter (Generics.X).  Calling it on a node class or
    instance returns the value bound to it there (None while open)."""

    def __init__(self, name: str) -> None:
        self.__name__ = name

    def __call__(self, obj):
        return generic_value(obj, self.__name__)

    def __repr__(self) -> str:
        return f"Generics.{self.__name__}"


class _GenericsNamespace:
    """Generics.X -> the (cached) parameter named X."""

    def __init__(self) -> None:
        self._params: dict[str, GenericParam] = {}
        self._lock = _threading.Lock()

    def __getattr__(self, name: str) -> GenericParam:
        if name.startswith("__"):
            raise AttributeError(name)
        with self._lock:
            p = self._params.get(name)
            if p is None:
                p = self._params[name] = GenericParam(name)
            return p


Generics = _GenericsNamespace()
IN = Generics.IN
OUT = Generics.OUT


class _GenericDeclaration:
    """Marker base produced by Generic[...]: the parameters a class declares."""

    __rdv_declares__: tuple = ()


class Generic:
    """Generic[P1, P2, ...] as a base class declares those parameters."""

    _cache: dict = {}

    def __class_getitem__(cls, params):
        if not isinstance(params, tuple):
            params = (params,)
        for p in params:
            if not isinstance(p, GenericParam):
                raise TypeError(f"Generic[...] takes generic parameters (Generics.X), got {p!r}")
        key = tuple(p.__name__ for p in params)
        if len(set(key)) != len(key):
            raise TypeError(f"Generic[...] declares a parameter twice: {key}")
        decl = cls._cache.get(key)
        if decl is None:
            decl = type(f"Generic[{', '.join(key)}]", (_GenericDeclaration,), {"__rdv_declares__": key})
            cls._cache[key] = decl
        return decl


def generic_value(obj, name: str):
    """Value bound to parameter `name` on a node class or instance (an
    instance's own shape attribute, e.g. a Map's IN, counts when its class
    leaves the parameter open)."""
    cls = obj if isinstance(obj, type) else type(obj)
    gens = getattr(cls, "__generics__", {})
    v = gens.get(name)
    if v is None:
        a = getattr(obj, name, None)
        if isinstance(a, (int, type)) and not isinstance(a, bool):
            v = a
    return v


# =============================================================== node meta

_UNSET = object()


def _resolve_template(template, bindings: dict):
    """An alias value with its generic parameters replaced by `bindings`:
    a parameter itself, or a subscripted type built from parameters."""
    if isinstance(template, GenericParam):
        v = bindings.get(template.__name__)
        return template if v is None else v
    args = getattr(template, "__rdv_type_args__", None)
    if args is not None:
        new = tuple(_resolve_template(a, bindings) for a in args)
        if new != args:
            return template.__rdv_type_origin__[new if len(new) > 1 else new[0]]
    return template


class _NodeMeta(type):
    """Metaclass of every node: collects declared generics and aliases,
    builds (cached) specialisations on subscription, and re-types an
    instance to the specialisation its constructor's match() calls bind."""

    def __new__(mcls, name, bases, dct, **kw):
        declared: list[str] = []
        for b in bases:
            if isinstance(b, type) and issubclass(b, _GenericDeclaration) and not isinstance(b, _NodeMeta):
                declared.extend(b.__rdv_declares__)
        inherited: dict = {}
        alias_templates: dict = {}
        for b in bases:
            for k, v in getattr(b, "__generics__", {}).items():
                if k not in inherited or inherited[k] is None:
                    inherited[k] = v
            for k, v in getattr(b, "__rdv_alias_templates__", {}).items():
                alias_templates.setdefault(k, v)
        for p in declared:
            if p in inherited:
                raise TypeError(f"{name}: generic parameter {p} is already declared by a base class")
        own_aliases = dct.get("__aliases__", {})
        new_aliases = {}
        for k, v in own_aliases.items():
            kname = k.__name__ if isinstance(k, GenericParam) else str(k)
            if kname in declared or kname in inherited:
                raise TypeError(f"{name}: {kname} is a generic parameter and cannot also be an alias")
            if kname in alias_templates and dct.get("__rdv_specialisation__") is None:
                raise TypeError(f"{name}: alias {kname} is already defined by a base class")
            new_aliases[kname] = v
        dct = dict(dct)
        dct.pop("__aliases__", None)
        cls = super().__new__(mcls, name, bases, dct, **kw)
        gens = dict(inherited)
        for p in declared:
            gens[p] = None
        if dct.get("__rdv_specialisation__") is not None:
            gens.update(dct["__rdv_specialisation__"])
        cls.__generics__ = gens
        alias_templates = {**alias_templates, **new_aliases}
        cls.__rdv_alias_templates__ = alias_templates
        cls.__aliases__ = {k: _resolve_template(v, gens) for k, v in alias_templates.items()}
        cls.__is_generic__ = any(v is None for v in gens.values())
        if "__rdv_origin__" not in dct:
            cls.__rdv_origin__ = cls
        cls.__rdv_specs__ = {}
        return cls

    # ------------------------------------------------------------ binding
    def _bindings_from_key(cls, key) -> dict:
        items = key if isinstance(key, tuple) else (key,)
        gens = cls.__generics__
        open_names = [k for k, v in gens.items() if v is None]
        out: dict = {}
        pos = 0
        for it in items:
            if isinstance(it, slice):
                p = it.start
                name = p.__name__ if isinstance(p, GenericParam) else p
                if not isinstance(name, str):
                    raise TypeError(f"{cls.__name__}[...]: a named binding needs a parameter name, got {p!r}")
                if name in cls.__aliases__:
                    raise TypeError(f"{cls.__name__}: {name} is an alias, not a generic parameter")
                if name not in gens:
                    raise TypeError(f"{cls.__name__} has no generic parameter {name}")
                out[name] = it.stop
            else:
                if isinstance(it, GenericParam):
                    raise TypeError(f"{cls.__name__}[{it!r}]: generic parameters are declared with "
                                    f"Generic[...], not by subscripting")
                while pos < len(open_names) and open_names[pos] in out:
                    pos += 1
                if pos >= len(open_names):
                    raise TypeError(f"{cls.__name__}: too many generic arguments")
                out[open_names[pos]] = it
                pos += 1
        for k, v in out.items():
            cur = gens.get(k)
            if cur is not None and v is not None and cur != v:
                raise TypeError(f"{cls.__name__}: generic {k} is already bound to {cur!r}, cannot bind {v!r}")
        return out

    def __getitem__(cls, key):
        return cls.specialise(cls._bindings_from_key(key))

    def specialise(cls, bindings: dict):
        """The subclass of `cls` with `bindings` added (cached per origin and
        binding set); `cls` itself when nothing new is bound."""
        gens = dict(cls.__generics__)
        changed = False
        for k, v in bindings.items():
            if v is not None and gens.get(k) is None:
                gens[k] = v
                changed = True
        if not changed:
            return cls
        key = tuple((k, _hashable(v)) for k, v in gens.items())
        hit = cls.__rdv_specs__.get(key)
        if hit is not None:
            return hit
        origin = cls.__rdv_origin__
        base_name = origin.__name__
        label = ", ".join(f"{k}={_short(v)}" for k, v in gens.items() if v is not None)
        spec = _NodeMeta(f"{base_name}[{label}]", (cls,), {
            "__rdv_specialisation__": {k: v for k, v in gens.items() if v is not None},
            "__rdv_origin__": origin,
            "__module__": cls.__module__,
            "__qualname__": f"{base_name}[{label}]",
        })
        cls.__rdv_specs__[key] = spec
        return spec

    def __instancecheck__(cls, obj):
        if type.__instancecheck__(cls, obj):
            return True
        origin = cls.__dict__.get("__rdv_origin__", cls)
        if origin is cls or not type.__instancecheck__(origin, obj):
            return False
        return all(generic_value(obj, k) == v for k, v in cls.__generics__.items() if v is not None)

    def __subclasscheck__(cls, sub):
        if type.__subclasscheck__(cls, sub):
            return True
        origin = cls.__dict__.get("__rdv_origin__", cls)
        if origin is cls or not isinstance(sub, type) or not type.__subclasscheck__(origin, sub):
            return False
        sg = getattr(sub, "__generics__", {})
        return all(sg.get(k) == v for k, v in cls.__generics__.items() if v is not None)

    # ------------------------------------------------------- construction
    def __call__(cls, *args, **kwargs):
        obj = cls.__new__(cls)
        obj.__dict__["_rdv_ctor"] = (args, kwargs)
        obj.__dict__["_rdv_pending"] = {}
        obj.__init__(*args, **kwargs)
        pending = obj.__dict__.pop("_rdv_pending", {})
        if pending:
            spec = type(obj).specialise(pending)
            if spec is not type(obj):
                obj.__class__ = spec
        return obj


def _hashable(v):
    try:
        hash(v)
        return v
    except TypeError:
        return id(v)


def _short(v) -> str:
    if isinstance(v, type):
        return v.__name__
    return repr(v)


class Node(metaclass=_NodeMeta):
    """Base of every rdv node (reference: _core.py Node)."""

    __requires__: list = []

    def match(self, param, value) -> None:
        """Binds generic `param` of this instance's class to `value` (from
        constructor data); a conflicting value raises TypeError."""
        name = param.__name__ if isinstance(param, GenericParam) else str(param)
        cls = type(self)
        if name not in cls.__generics__:
            raise TypeError(f"{cls.__name__} has no generic parameter {name}")
        cur = cls.__generics__.get(name)
        if cur is not None:
            if value is not None and cur != value:
                raise TypeError(f"{cls.__name__}: generic {name} is {cur!r}, cannot match {value!r}")
            return
        pending = self.__dict__.setdefault("_rdv_pending", {})
        prev = pending.get(name)
        if prev is not None and value is not None and prev != value:
            raise TypeError(f"{cls.__name__}: generic {name} matched to both {prev!r} and {value!r}")
        if value is not None:
            pending[name] = value

    def cast(self, target):
        """This node rebound to `target`, a (partial) specialisation of one
        of its own base classes: the shared parameters must agree; the
        constructor is replayed on the resulting specialisation of this
        node's own class.  Casting to the bindings it already has returns
        an equal node; an unrelated target raises TypeError."""
        cls = type(self)
        origin = target.__dict__.get("__rdv_origin__", target) if isinstance(target, type) else None
        if origin is None or not issubclass(cls, origin):
            raise TypeError(f"cannot cast {cls.__name__} to unrelated type {getattr(target, '__name__', target)}")
        want = {k: v for k, v in getattr(target, "__generics__", {}).items() if v is not None}
        for k, v in want.items():
            cur = generic_value(self, k)
            if cur is not None and cur != v:
                raise TypeError(f"cannot cast {cls.__name__}: generic {k} is {cur!r}, target needs {v!r}")
        spec = cls.specialise(want)
        if spec is cls:
            return self
        args, kwargs = self.__dict__.get("_rdv_ctor", ((), {}))
        return spec(*args, **kwargs)


class Component(Node):
    """A node with fields (reference: _core.py Component)."""


class Struct(Node):
    """A plain data node (reference: _core.py Struct)."""


class Main(Component):
    """A dispatchable root node (reference: _core.py Main): dispatch(main, ...)
    launches its work through the HIP library."""

    def _dispatch(self, threads: int) -> None:
        raise NotImplementedError(f"{type(self).__name__} has no dispatch")


class Library(Node):
    """A node that only contributes shared code in the reference; here a
    namespace for host-side state (reference: _core.py Library)."""


class Code(Node):
    """A trait node (reference: _core.py Code)."""


class MathLibrary(Library):
    """Shared maths (math_library.h: ray_box_intersection etc.); its
    functions live in the kernels here (reference: _common.py:51)."""


class CooperativeLibrary(Library):
    """Workgroup cooperation helpers (cooperative_library.h); the matrix-core
    kernels here tile uniformly by construction (reference: _common.py:92)."""


class GridLibrary(Library):
    """Row-major grid index helpers (grid_library.h; reference: _common.py:97)."""


class RandomLibrary(Library):
    """Per-dispatch random seeds (reference: _common.py:56-89): every dispatch
    that draws random numbers gets a fresh uvec4 of integers in [128, 2^30)
    from a host generator; seed(s) makes that sequence reproducible."""

    _lock = _threading.Lock()
    _rng = None

    @classmethod
    def seed(cls, s: int | None) -> None:
        import random as _random
        with cls._lock:
            cls._rng = _random.Random(s)

    @classmethod
    def next_seeds(cls) -> tuple:
        import random as _random
        with cls._lock:
            if cls._rng is None:
                cls._rng = _random.Random()
            return tuple(cls._rng.randint(128, 1 << 30) for _ in range(4))


def _dependency_order(root) -> list:
    """Post-order of root's __requires__ graph: every node after all it
    requires, each once (reference: _core.py:1578-1614)."""
    order: list = []
    state: dict = {}  # id -> 1 visiting, 2 done
    stack = [(root, iter(list(getattr(root, "__requires__", []))))]
    state[id(root)] = 1
    while stack:
        node, it = stack[-1]
        nxt = next(it, _UNSET)
        if nxt is _UNSET:
            stack.pop()
            state[id(node)] = 2
            order.append(node)
            continue
        s = state.get(id(nxt))
        if s == 2:
            continue
        if s == 1:
            raise ValueError(f"dependency cycle through {nxt!r}")
        state[id(nxt)] = 1
        stack.append((nxt, iter(list(getattr(nxt, "__requires__", [])))))
    return order


# ============================================================ value types


class Type(_enum.Enum):
    """Scalar element types (reference: vulky's Type as re-exported by rdv)."""
    FLOAT32 = "float"
    FLOAT16 = "float16_t"
    FLOAT64 = "double"
    INT32 = "int"
    INT64 = "int64_t"
    UINT32 = "uint"
    UINT64 = "uint64_t"
    BOOL = "bool"
    UVEC4 = "uvec4"


class _TypeOp:
    """Type constructors T[...] with identity-cached results, so that
    Pointer[vec3] is Pointer[vec3] (the reference's alias tests rely on it)."""

    def __init__(self, name: str, arity: int) -> None:
        self.__name__ = name
        self._arity = arity
        self._cache: dict = {}
        self._lock = _threading.Lock()

    def __getitem__(self, args):
        if not isinstance(args, tuple):
            args = (args,)
        if len(args) != self._arity:
            raise TypeError(f"{self.__name__}[...] takes {self._arity} argument(s)")
        key = tuple(_hashable(a) for a in args)
        with self._lock:
            hit = self._cache.get(key)
            if hit is None:
                label = ", ".join(_short(a) for a in args)
                hit = type(f"{self.__name__}[{label}]", (_TypeInstance,), {
                    "__rdv_type_origin__": self, "__rdv_type_args__": args})
                self._cache[key] = hit
            return hit

    def __repr__(self) -> str:
        return self.__name__


class _TypeInstance:
    __rdv_type_origin__ = None
    __rdv_type_args__: tuple = ()


Single = _TypeOp("Single", 1)
Array = _TypeOp("Array", 2)
Pointer = _TypeOp("Pointer", 1)
Buffer = _TypeOp("Buffer", 1)
FixArray = _TypeOp("FixArray", 2)
_DeferredType = _TypeOp("Deferred", 1)


# --------------------------------------------------------------- deferreds


class DeferredLibrary(Library):
    """Name -> object bindings visible while a call runs (reference:
    _common.py:100-167; there a pointer table in a storage buffer)."""

    _local = _threading.local()

    @classmethod
    def _table(cls) -> dict:
        t = getattr(cls._local, "table", None)
        if t is None:
            t = cls._local.table = {}
        return t

    @classmethod
    def bind(cls, **deferreds) -> None:
        cls._table().update(deferreds)

    @classmethod
    def unbind(cls, **deferreds) -> None:
        t = cls._table()
        for k in deferreds:
            t.pop(k, None)

    @classmethod
    def lookup(cls, name: str):
        t = cls._table()
        if name not in t:
            raise RuntimeError(f"deferred '{name}' is not bound (pass it as a keyword to the call, or use "
                               f"`with deferreds({name}=...)`)")
        return t[name]


class Deferred:
    """A field value resolved at dispatch: Deferred(name) is looked up among
    the names bound for the current call, Deferred(obj=x) is x itself
    (reference: _common.py:234-279).  Deferred[T] is the field type."""

    def __class_getitem__(cls, t):
        return _DeferredType[t]

    def __init__(self, name: str | None = None, offset: int | None = None, obj=None) -> None:
        assert name is not None or (obj is not None and offset is not None) or obj is not None, \
            "Either name or obj must be provided. Offset is valid only if deferred."
        self.name = name
        self.offset = 0 if offset is None else int(offset)
        self.obj = obj

    def resolve(self):
        return self.obj if self.obj is not None else DeferredLibrary.lookup(self.name)

    def __repr__(self) -> str:
        return f"Deferred({self.name!r})" if self.obj is None else f"Deferred(obj={self.obj!r})"


def resolve(value):
    """A Deferred's bound object, anything else unchanged."""
    return value.resolve() if isinstance(value, Deferred) else value


class _DeferredContext:
    def __init__(self, **deferreds) -> None:
        self._deferreds = deferreds

    def __enter__(self):
        DeferredLibrary.bind(**self._deferreds)
        return self

    def __exit__(self, exc_type, exc, tb):
        DeferredLibrary.unbind(**self._deferreds)


def deferreds(**deferreds):
    """`with deferreds(name=tensor): ...` binds names for the calls inside
    (reference: _common.py:282-311)."""
    return _DeferredContext(**deferreds)


# ============================================================ GLSL vectors


class _VecBase:
    """A small fixed-size GLSL vector (component access x, y, z, w)."""

    _n = 0
    _kind = float
    __slots__ = ("_v",)

    def __init__(self, *args) -> None:
        vals: list = []
        for a in args:
            if isinstance(a, (_VecBase, _MatBase)):
                vals.extend(a.tolist_flat())
            elif isinstance(a, (list, tuple)):
                vals.extend(a)
            elif hasattr(a, "tolist") and not isinstance(a, (int, float)):
                t = a.tolist()
                vals.extend(t if isinstance(t, list) else [t])
            else:
                vals.append(a)
        if len(vals) == 1 and self._n > 1:
            vals = vals * self._n
        if len(vals) == 0:
            vals = [0] * self._n
        if len(vals) != self._n:
            raise ValueError(f"{type(self).__name__} needs {self._n} components, got {len(vals)}")
        self._v = [self._kind(v) for v in vals]

    def tolist_flat(self) -> list:
        return list(self._v)

    def __len__(self) -> int:
        return self._n

    def __iter__(self):
        return iter(self._v)

    def __getitem__(self, i):
        return self._v[i]

    def __setitem__(self, i, v) -> None:
        self._v[i] = self._kind(v)

    def __eq__(self, other) -> bool:
        return isinstance(other, _VecBase) and type(other) is type(self) and other._v == self._v

    def __hash__(self):
        return hash((type(self).__name__, tuple(self._v)))

    def __repr__(self) -> str:
        return f"{type(self).__name__}({', '.join(map(repr, self._v))})"

    x = property(lambda self: self._v[0], lambda self, v: self.__setitem__(0, v))
    y = property(lambda self: self._v[1], lambda self, v: self.__setitem__(1, v))
    z = property(lambda self: self._v[2], lambda self, v: self.__setitem__(2, v))
    w = property(lambda self: self._v[3], lambda self, v: self.__setitem__(3, v))


def _vec(name: str, n: int, kind):
    return type(name, (_VecBase,), {"_n": n, "_kind": kind, "__slots__": ()})


vec2, vec3, vec4 = _vec("vec2", 2, float), _vec("vec3", 3, float), _vec("vec4", 4, float)
ivec2, ivec3, ivec4 = _vec("ivec2", 2, int), _vec("ivec3", 3, int), _vec("ivec4", 4, int)
uvec2, uvec3, uvec4 = _vec("uvec2", 2, int), _vec("uvec3", 3, int), _vec("uvec4", 4, int)
bvec2, bvec3, bvec4 = _vec("bvec2", 2, bool), _vec("bvec3", 3, bool), _vec("bvec4", 4, bool)


class _MatBase:
    """A GLSL matColsxRows matrix, column-major: mat4x3 is 4 columns of vec3;
    built from cols * rows floats in column order (or another matrix of the
    same shape)."""

    _cols = 0
    _rows = 0
    __slots__ = ("_v",)

    def __init__(self, *args) -> None:
        vals: list = []
        for a in args:
            if isinstance(a, (_VecBase, _MatBase)):
                vals.extend(a.tolist_flat())
            elif isinstance(a, (list, tuple)):
                for e in a:
                    vals.extend(e.tolist_flat() if isinstance(e, (_VecBase, _MatBase)) else
                                (list(e) if isinstance(e, (list, tuple)) else [e]))
            elif hasattr(a, "reshape") and hasattr(a, "tolist"):
                vals.extend(a.reshape(-1).tolist())
            else:
                vals.append(a)
        n = self._cols * self._rows
        if len(vals) == 1:  # diagonal
            d = float(vals[0])
            vals = [d if c == r else 0.0 for c in range(self._cols) for r in range(self._rows)]
        if len(vals) == 0:
            vals = [1.0 if c == r else 0.0 for c in range(self._cols) for r in range(self._rows)]
        if len(vals) != n:
            raise ValueError(f"{type(self).__name__} needs {n} values, got {len(vals)}")
        self._v = [float(v) for v in vals]

    def tolist_flat(self) -> list:
        """Column-major flat values."""
        return list(self._v)

    def column(self, c: int) -> list:
        return self._v[c * self._rows:(c + 1) * self._rows]

    def __getitem__(self, c):
        return self.column(c)

    def __len__(self) -> int:
        return self._cols

    def __iter__(self):
        return iter(self.column(c) for c in range(self._cols))

    def __eq__(self, other) -> bool:
        return isinstance(other, _MatBase) and type(other) is type(self) and other._v == self._v

    def __hash__(self):
        return hash((type(self).__name__, tuple(self._v)))

    def __repr__(self) -> str:
        return f"{type(self).__name__}({', '.join(map(repr, self._v))})"


def _mat(name: str, cols: int, rows: int):
    return type(name, (_MatBase,), {"_cols": cols, "_rows": rows, "__slots__": ()})


mat2, mat3, mat4 = _mat("mat2", 2, 2), _mat("mat3", 3, 3), _mat("mat4", 4, 4)
mat3x4, mat4x3 = _mat("mat3x4", 3, 4), _mat("mat4x3", 4, 3)


# ================================================================ dispatch

_dispatch_count = _itertools.count()


def dispatch(main: Main, tx: int = 1, ty: int = 1, tz: int = 1) -> None:
    """Runs `main` over tx * ty * tz threads and waits for it, as the
    reference's synchronous dispatch does (_core.py:2799-2886).  `main` is
    one of this build's evaluators (MapEvaluator, GridEvaluator,
    TensorOpEvaluator), each of which launches its HIP kernels."""
    from .core import launch_scope
    if not isinstance(main, Main):
        raise TypeError(f"dispatch needs a Main node, got {type(main).__name__}")
    next(_dispatch_count)
    with launch_scope():
        main._dispatch(int(tx) * int(ty) * int(tz))
