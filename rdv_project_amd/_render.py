"""Grid evaluation and the rendering kernels through the C ABI
(rdv_cameras_rays, rdv_render_emission_absorption, rdv_composite,
rdv_raymarch_transmittance).

Reference: Grid.__call__ (src/rdv/maths/__init__.py:77-103) evaluates every cell
of a grid in row-major order into a per-class cached [*shape, OUT] buffer; a
Sensor (maths:252-271) applies its map to each cell's value.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _chain, _lib
from .core import RDVObject, current_stream_handle, device, launch_scope, wrap
from .maths import Grid, Sensor
from .rendering import Cameras, EmissionAbsorption, RaymarchingTransmittance

_GRID_CACHE: dict = {}


def _cached(key, shape) -> RDVObject:
    hit = _GRID_CACHE.get(key)
    if hit is not None and hit[0] == tuple(shape):
        return hit[1]
    out = RDVObject(torch.empty(tuple(shape), dtype=torch.float32, device=device()))
    _GRID_CACHE[key] = (tuple(shape), out)
    return out


def camera_desc(cam: Cameras) -> _lib.CameraDesc:
    d = _lib.CameraDesc()
    d.n_cams, d.width, d.height = cam.shape[0], cam.width, cam.height
    d.aspect_ratio, d.fov = cam.aspect_ratio, cam.fov
    return d


def _poses(cam: Cameras) -> torch.Tensor:
    p = cam.poses.as_tensor("torch")
    if p.dtype != torch.float32 or not p.is_contiguous():
        p = p.to(torch.float32).contiguous()
    return p


def camera_rays(cam: Cameras, out: RDVObject | None = None) -> RDVObject:
    n, H, W = cam.shape
    out = out if out is not None else _cached(("cameras",), (n, H, W, 6))
    d = camera_desc(cam)
    with launch_scope():
        _lib.check(_lib.load().rdv_cameras_rays(C.byref(d), C.c_void_p(_poses(cam).data_ptr()),
                                                C.c_void_p(out.device_ptr), C.c_void_p(current_stream_handle())),
                   "Cameras")
    return out


def _field_plan(m, in_width: int):
    p = _chain.plan_chain(m, in_width)
    return p, _chain.packed_params(m, p)


def render_ea(cam: Cameras, ea: EmissionAbsorption, out: RDVObject | None = None) -> RDVObject:
    n, H, W = cam.shape
    out = out if out is not None else _cached(("ea",), (n, H, W, 3))
    p, packed = _field_plan(ea.field, 3)
    d = camera_desc(cam)
    with launch_scope():
        _lib.check(_lib.load().rdv_render_emission_absorption(
            C.byref(d), C.c_void_p(_poses(cam).data_ptr()), C.byref(p.desc), C.c_void_p(packed.data_ptr()),
            C.c_int32(ea.samples), C.c_void_p(out.device_ptr), C.c_void_p(current_stream_handle())),
            "EmissionAbsorption")
    return out


def render_ea_rays(ea: EmissionAbsorption, rays_ptr: int, out_ptr: int, n_rays: int) -> None:
    """EmissionAbsorption over n_rays rays (fp32 [n, 6] at rays_ptr) into fp32
    [n, 3] at out_ptr: the renderer with rays read from memory."""
    p, packed = _field_plan(ea.field, 3)
    _lib.check(_lib.load().rdv_render_emission_absorption_rays(
        C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.c_void_p(rays_ptr), C.c_int64(n_rays),
        C.c_int32(ea.samples), C.c_void_p(out_ptr), C.c_void_p(current_stream_handle())), "EmissionAbsorption")


def _transform_array(rt: RaymarchingTransmittance):
    arr = (C.c_float * 12)()
    for i, v in enumerate(rt.transform.tolist_flat()):
        arr[i] = v
    return arr


def raymarch_ptrs(rt: RaymarchingTransmittance, x_ptr: int, y_ptr: int, rows: int) -> None:
    """RaymarchingTransmittance over `rows` rays (fp32 [rows, 6] at x_ptr) into
    fp32 [rows] at y_ptr."""
    p, packed = _field_plan(rt.extinction, 3)
    _lib.check(_lib.load().rdv_raymarch_transmittance(
        C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.c_void_p(x_ptr), C.c_int64(rows), _transform_array(rt),
        C.c_float(rt.step_size), C.c_float(rt.density_scale), C.c_void_p(y_ptr),
        C.c_void_p(current_stream_handle())), "RaymarchingTransmittance")


def raymarch_rows(rt: RaymarchingTransmittance, x, out: RDVObject | None = None) -> RDVObject:
    """RaymarchingTransmittance over rows x [..., 6] -> [..., 1]."""
    x = wrap(x)
    if x.scalar_type != torch.float32:
        raise TypeError(f"Map input must be float32, got {x.scalar_type}")
    assert x.shape[-1] == 6, "RaymarchingTransmittance expects rows of 6 values (x, w)"
    rows = 1
    for s in x.shape[:-1]:
        rows *= int(s)
    out = out if out is not None else _cached(("rt", id(type(rt))), (*x.shape[:-1], 1))
    p, packed = _field_plan(rt.extinction, 3)
    xt = x.as_tensor("torch")
    if not xt.is_contiguous():
        xt = xt.contiguous()
    with launch_scope():
        _lib.check(_lib.load().rdv_raymarch_transmittance(
            C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.c_void_p(xt.data_ptr()), C.c_int64(rows),
            _transform_array(rt), C.c_float(rt.step_size), C.c_float(rt.density_scale), C.c_void_p(out.device_ptr),
            C.c_void_p(current_stream_handle())), "RaymarchingTransmittance")
    return out


def composite(sigma_rgb: torch.Tensor, dt: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Front-to-back compositing of samples sigma_rgb [n_rays, S, 4] = (sigma,
    r, g, b) with spacing dt [n_rays] -> [n_rays, 3] (build-defined)."""
    assert sigma_rgb.dim() == 3 and sigma_rgb.shape[2] == 4, "sigma_rgb must be [n_rays, samples, 4]"
    n, S = int(sigma_rgb.shape[0]), int(sigma_rgb.shape[1])
    s = sigma_rgb.to(device=device(), dtype=torch.float32).contiguous()
    d = dt.to(device=device(), dtype=torch.float32).contiguous()
    assert tuple(d.shape) == (n,), "dt must be [n_rays]"
    if out is None:
        out = torch.empty((n, 3), dtype=torch.float32, device=device())
    else:
        if not isinstance(out, torch.Tensor) or out.device.type != "cuda":
            raise TypeError("out must be a GPU tensor")
        assert out.dtype == torch.float32 and tuple(out.shape) == (n, 3) and out.is_contiguous(), \
            "out must be a contiguous float32 [n_rays, 3] tensor"
    with launch_scope():
        _lib.check(_lib.load().rdv_composite(C.c_void_p(s.data_ptr()), C.c_void_p(d.data_ptr()), C.c_int64(n),
                                             C.c_int32(S), C.c_void_p(out.data_ptr()),
                                             C.c_void_p(current_stream_handle())), "composite")
    return out


def evaluate_grid(g: Grid, out: RDVObject | None = None) -> RDVObject:
    if isinstance(g, Cameras):
        return camera_rays(g, out)
    if isinstance(g, Sensor) and isinstance(g.grid, Cameras):
        cam, m = g.grid, g.map
        if isinstance(m, EmissionAbsorption):
            return render_ea(cam, m, out)
        rays = camera_rays(cam, _cached(("sensor-rays",), (*cam.shape, 6)))
        if isinstance(m, RaymarchingTransmittance):
            return raymarch_rows(m, rays, out if out is not None else _cached(("sensor-rt",), (*cam.shape, 1)))
        y = m(rays)
        if out is not None:
            out.as_tensor("torch").copy_(y.as_tensor("torch").reshape(out.shape))
            return out
        return y
    # any other grid graph: node by node (grids.py)
    from .grids import grid_values
    with launch_scope():
        v = grid_values(g, {})
    if out is not None:
        out.as_tensor("torch").copy_(v.as_tensor("torch").reshape(out.shape))
        return out
    return v
