"""Device objects, profiling counters and launch semantics of the rdv API.

Mirrors, for the hot path only:
  - RDVObject / wrap      src/rdv/core/_core.py:273-380
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
import time as _time

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
    _core.py:278-284); wrapping a contiguous GPU tensor is zero-copy.
    """

    def __init__(self, data):
        self._data = data
        self._t = _as_device_tensor(data)
        self._direct = isinstance(data, torch.Tensor) and data.device.type == "cuda" and data.is_contiguous()

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

    def update_device(self) -> None:
        """Re-uploads the wrapped host data (non-direct objects only)."""
        if not self._direct:
            self._t.copy_(torch.as_tensor(self._data).to(self._t.dtype))

    def host(self) -> "RDVObject":
        return RDVObject(self._t.detach().cpu())

    def device(self) -> "RDVObject":
        return RDVObject(self._t.clone())

    def __repr__(self) -> str:
        return f"RDVObject(shape={self.shape}, dtype={self.scalar_type}, device={self._t.device})"


def wrap(data) -> RDVObject:
    if isinstance(data, RDVObject):
        return data
    return RDVObject(data)


def is_on_rdv(data) -> bool:
    return isinstance(data, RDVObject) or (isinstance(data, torch.Tensor) and data.device.type == "cuda")


def ensure_on_rdv(data) -> RDVObject:
    return wrap(data)
