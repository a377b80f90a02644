"""Device objects, profiling counters and launch semantics of the rdv API.

Mirrors, for the hot path only:
  - RDVObject / wrap      src/rdv/core/_core.py:273-380
  - is_on_rdv / ensure_on_rdv, MemoryLocation
                          src/rdv/core/_common.py:330-439
  - profiling(), reset_submit_times(), profiling_submit_times()
                          src/rdv/core/_core.py:54-59, 3179-3188
  - dispatch's synchronous submit (`vk.submit_and_wait`, _core.py:2877-2886):
    every launch made through this package waits for completion unless
    set_synchronous(False) was called; with profiling on, the wall time of each
    launch + wait is added to the submit-time counter exactly as the reference
    times `submit_and_wait`.

Device memory is PyTorch-ROCm's (one GPU, torch's current device and stream).
"""
from __future__ import annotations

import contextlib
import enum
import time as _time
import weakref

import torch

__PROFILING__ = False
__submit_times__ = 0.0
__SYNCHRONOUS__ = True


def profiling(enable: bool = True) -> None:
    """Turns the submit-time counter on or off (reference: _core.py:57-59)."""
    global __PROFILING__
    __PROFILING__ = bool(enable)


def reset_submit_times() -> None:
    global __submit_times__
    __submit_times__ = 0.0


def profiling_submit_times() -> float:
    """Seconds spent in launches (+ waits) since the last reset."""
    return __submit_times__


def set_synchronous(enable: bool) -> bool:
    """Whether every launch waits for completion (the reference always does).
    Returns the previous setting.  Turning it off leaves launches ordered on
    torch's current stream, which is how a stream-aware caller wants them."""
    global __SYNCHRONOUS__
    prev = __SYNCHRONOUS__
    __SYNCHRONOUS__ = bool(enable)
    return prev


def device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("rdv_project_amd needs a ROCm GPU: torch.cuda.is_available() is False")
    return torch.device("cuda", torch.cuda.current_device())


def current_stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


@contextlib.contextmanager
def launch_scope():
    """Wraps one logical dispatch: optional wait + profiling, as `dispatch` does."""
    global __submit_times__
    t0 = _time.perf_counter() if __PROFILING__ else 0.0
    yield
    if __SYNCHRONOUS__:
        torch.cuda.current_stream().synchronize()
    if __PROFILING__:
        __submit_times__ += _time.perf_counter() - t0


def _as_device_tensor(data) -> torch.Tensor:
    """Contiguous GPU copy/view of `data`.  Without a GPU the data stays in host
    memory so that graph construction and validation still work; every launch
    path then fails in device()."""
    if isinstance(data, RDVObject):
        return data._t
    if isinstance(data, torch.Tensor):
        t = data
    else:
        t = torch.as_tensor(data)
        if t.dtype == torch.float64:
            t = t.to(torch.float32)
    if t.device.type != "cuda" and torch.cuda.is_available():
        t = t.to(device())
    return t.contiguous()


class RDVObject:
    """A device tensor as rdv sees it: shape, scalar type and a device pointer.

    Wrapping host data copies it to the GPU (the reference's non-direct case,
    _core.py:278-284); wrapping a contiguous GPU tensor is zero-copy.  For a
    non-direct object the host data and the device copy are kept apart:
    update_device() uploads the host data, update_host() writes the device
    copy back into the wrapped host array or tensor, in place.
    make_host_dirty() / make_device_dirty() record which side was written
    last: an update does not overwrite the side marked as the newer one, and
    copies whenever neither (or both) is marked.  Each update clears both
    marks.
    """

    def __init__(self, data):
        self._data = data
        self._t = _as_device_tensor(data)
        self._direct = isinstance(data, torch.Tensor) and data.device.type == "cuda" and data.is_contiguous()
        self._host_dirty = False
        self._device_dirty = False

    @property
    def device_ptr(self) -> int:
        return self._t.data_ptr()

    @property
    def shape(self):
        return tuple(self._t.shape)

    @property
    def scalar_type(self):
        return self._t.dtype

    @property
    def is_direct(self) -> bool:
        return self._direct

    @property
    def device_index(self) -> int:
        return self._t.device.index

    def as_tensor(self, backend: str = "torch"):
        """A live view (torch) or a host copy (numpy) of this object's memory."""
        if backend == "torch":
            return self._t
        if backend == "numpy":
            return self._t.detach().cpu().numpy()
        raise NotImplementedError(f"Unknown backend {backend}. Supported backends here are: torch, numpy.")

    def make_host_dirty(self) -> None:
        """The wrapped host data was written (reference: _core.py:344-345)."""
        self._host_dirty = True

    def make_device_dirty(self) -> None:
        """The device copy was written, e.g. by a kernel (reference: _core.py:347-348)."""
        self._device_dirty = True

    def update_device(self) -> None:
        """Uploads the wrapped host data into the device copy (non-direct
        objects; reference: _core.py:353-354)."""
        if self._direct:
            return
        if not (self._device_dirty and not self._host_dirty):
            src = torch.as_tensor(self._data)
            self._t.copy_(src.reshape(self._t.shape).to(self._t.dtype))
        self._host_dirty = self._device_dirty = False

    def update_host(self) -> None:
        """Writes the device copy back into the wrapped host array or tensor, in
        place (non-direct objects; reference: _core.py:350-351)."""
        if self._direct:
            return
        if not (self._host_dirty and not self._device_dirty):
            if self._t.data_ptr() != _host_ptr(self._data):
                _write_back(self._data, self._t)
        self._host_dirty = self._device_dirty = False

    def host(self) -> "RDVObject":
        """A copy of this object's current data in host memory."""
        return RDVObject(self._t.detach().cpu().clone())

    def device(self) -> "RDVObject":
        """A copy of this object's current data in device memory."""
        return RDVObject(self._t.clone())

    def __repr__(self) -> str:
        return f"RDVObject(shape={self.shape}, dtype={self.scalar_type}, device={self._t.device})"


def _host_ptr(data) -> int:
    if isinstance(data, torch.Tensor):
        return data.data_ptr()
    ai = getattr(data, "__array_interface__", None)
    return int(ai["data"][0]) if ai else -1


def _write_back(data, t: torch.Tensor) -> None:
    """Copies device tensor t into host data (a numpy array or a torch tensor) in place."""
    if isinstance(data, torch.Tensor):
        data.copy_(t.reshape(data.shape).to(data.dtype))
        return
    import numpy as np
    if isinstance(data, np.ndarray):
        np.copyto(data, t.detach().cpu().numpy().reshape(data.shape), casting="unsafe")
        return
    raise TypeError(f"update_host cannot write into a {type(data).__name__}: wrap a numpy array or a tensor")


def wrap(data) -> RDVObject:
    if isinstance(data, RDVObject):
        return data
    return RDVObject(data)


class MemoryLocation(enum.Enum):
    """Where ensure_on_rdv places its copy (the reference re-exports vulky's
    MemoryLocation for this)."""
    HOST = "host"
    DEVICE = "device"


# Memory handed out by ensure_on_rdv, keyed by data pointer: a weak reference
# to the object returned, dropped when that object is collected.
_OWNED: dict = {}


def _own(obj, ptr: int) -> None:
    ref = weakref.ref(obj)
    _OWNED[ptr] = ref

    def _drop(p=ptr, r=ref):
        if _OWNED.get(p) is r:
            del _OWNED[p]
    weakref.finalize(obj, _drop)


def _data_ptr(data) -> int | None:
    if isinstance(data, torch.Tensor):
        return data.untyped_storage().data_ptr() if data.numel() else None
    ai = getattr(data, "__array_interface__", None)
    if ai is None:
        return None
    base = data
    while getattr(base, "base", None) is not None and hasattr(base.base, "__array_interface__"):
        base = base.base
    return int(base.__array_interface__["data"][0])


def is_on_rdv(data) -> bool:
    """Whether data's memory is already the library's own (reference:
    _common.py:357-378): an RDVObject that is direct, or a tensor / array whose
    memory ensure_on_rdv handed out (views of it included).  False for any
    other memory, GPU-resident or not."""
    if isinstance(data, RDVObject):
        return data.is_direct
    ptr = _data_ptr(data)
    if ptr is None:
        return False
    ref = _OWNED.get(ptr)
    return ref is not None and ref() is not None


_BACKENDS = {"torch": "torch", "numpy": "numpy"}


def _detect_backend(data) -> str:
    root = type(data).__module__.split(".")[0]
    backend = _BACKENDS.get(root)
    if backend is None:
        raise TypeError(f"ensure_on_rdv: could not infer a supported backend from {type(data)!r} "
                        f"(module {root!r}) - pass backend explicitly.")
    return backend


def _infer_location(data) -> MemoryLocation:
    if isinstance(data, torch.Tensor):
        return MemoryLocation.HOST if data.device.type == "cpu" else MemoryLocation.DEVICE
    if hasattr(data, "__array_interface__"):
        return MemoryLocation.HOST
    return MemoryLocation.DEVICE


def ensure_on_rdv(data, backend: str | None = None, location: MemoryLocation | None = None):
    """`data` itself if is_on_rdv(data), else a copy of it in fresh memory that
    the library owns, returned as the same backend type as `data` (or
    `backend`: 'torch' or 'numpy') -- not a view of the caller's memory
    (reference: _common.py:381-439).  location defaults to where data lives
    (HOST for numpy and CPU tensors); a numpy result cannot live on the device:
    with backend='numpy' and location=DEVICE this raises ValueError, with the
    backend inferred the copy becomes a torch tensor."""
    if is_on_rdv(data):
        return data
    backend_given = backend is not None
    if backend is None:
        backend = _detect_backend(data)
    if backend not in ("torch", "numpy"):
        raise NotImplementedError(f"Unknown backend {backend}. Supported backends here are: torch, numpy.")
    if location is None:
        location = _infer_location(data)
    if location == MemoryLocation.DEVICE and backend == "numpy":
        if backend_given:
            raise ValueError(f"ensure_on_rdv: backend={backend!r} can't represent DEVICE-resident memory - pass a "
                             "device-capable backend (e.g. 'torch') explicitly, or leave location unspecified/HOST.")
        backend = "torch"
    src = data._t if isinstance(data, RDVObject) else torch.as_tensor(data)
    shape = tuple(data.shape) if hasattr(data, "shape") else tuple(src.shape)
    if location == MemoryLocation.DEVICE:
        out = torch.empty(shape, dtype=src.dtype, device=device())
    else:
        out = torch.empty(shape, dtype=src.dtype)
    out.copy_(src.reshape(shape))
    if backend == "numpy":
        arr = out.numpy()
        _own(arr, _data_ptr(arr))
        return arr
    if out.numel():
        _own(out, _data_ptr(out))
    return out
