"""Grid evaluation and the rendering kernels through the C ABI
(rdv_cameras_rays, rdv_render_emission_absorption, rdv_composite,
rdv_raymarch_transmittance, rdv_ratiotracking_transmittance,
rdv_volume_profile).

Reference: Grid.__call__ (src/rdv/maths/__init__.py:77-103) evaluates every cell
of a grid in row-major order into a per-class cached [*shape, OUT] buffer; a
Sensor (maths:252-271) applies its map to each cell's value.  With a batch of
index vectors (maths:104-119, BatchGridEvaluator) only those cells are
evaluated, one thread per index vector (rdv_cameras_rays_at, rdv_grid_gather
and the map kernels over the gathered rows).
"""
from __future__ import annotations

import ctypes as C
import math

import torch

from . import _chain, _lib
from .core import RDVObject, current_stream_handle, device, launch_scope, wrap
from .maths import Grid, Sensor
from .rendering import (Cameras, EmissionAbsorption, RaymarchingTransmittance, RatiotrackingTransmittance,
                        VolumeProfile, VolumeProfileDDA, VoxelMajorantField)

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


def _seed_array(seeds):
    arr = (C.c_uint32 * 4)()
    for i, v in enumerate(seeds):
        arr[i] = int(v) & 0xFFFFFFFF
    return arr


def camera_rays(cam: Cameras, out: RDVObject | None = None, seeds=None) -> RDVObject:
    """The cameras' rays [n, H, W, 6].  A jittered camera draws with `seeds`
    (4 words; fresh RandomLibrary seeds when None)."""
    n, H, W = cam.shape
    out = out if out is not None else _cached(("cameras",), (n, H, W, 6))
    d = camera_desc(cam)
    lib = _lib.load()
    with launch_scope():
        if cam.pixel_jitter:
            from .types import RandomLibrary
            seeds = RandomLibrary.next_seeds() if seeds is None else seeds
            _lib.check(lib.rdv_cameras_rays_jittered(C.byref(d), C.c_void_p(_poses(cam).data_ptr()),
                                                     _seed_array(seeds), C.c_void_p(out.device_ptr),
                                                     C.c_void_p(current_stream_handle())), "Cameras")
        else:
            _lib.check(lib.rdv_cameras_rays(C.byref(d), C.c_void_p(_poses(cam).data_ptr()),
                                            C.c_void_p(out.device_ptr), C.c_void_p(current_stream_handle())),
                       "Cameras")
    return out


def random_uniform(seeds, n_threads: int, per_thread: int) -> torch.Tensor:
    """[n_threads, per_thread]: the first random() values of each thread of a
    dispatch with these seeds (the generator every random node draws from)."""
    out = torch.empty((n_threads, per_thread), dtype=torch.float32, device=device())
    with launch_scope():
        _lib.check(_lib.load().rdv_random_uniform(_seed_array(seeds), C.c_int64(n_threads), C.c_int32(per_thread),
                                                  C.c_void_p(out.data_ptr()), C.c_void_p(current_stream_handle())),
                   "random_uniform")
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


def _ray_rows(x, name: str, out_width: int, key) -> tuple[torch.Tensor, int, RDVObject]:
    x = wrap(x)
    if x.scalar_type != torch.float32:
        raise TypeError(f"Map input must be float32, got {x.scalar_type}")
    assert x.shape[-1] == 6, f"{name} expects rows of 6 values (x, w)"
    rows = 1
    for s_ in x.shape[:-1]:
        rows *= int(s_)
    xt = x.as_tensor("torch")
    if not xt.is_contiguous():
        xt = xt.contiguous()
    return xt, rows, _cached(key, (*x.shape[:-1], out_width))


def _grid_values_dhw(grid) -> tuple[torch.Tensor, int, int, int]:
    """A 3-D Grid[3, 1]'s values as a contiguous fp32 [D, H, W] tensor and (W, H, D)."""
    from .grids import grid_values
    D, H, W = (int(v) for v in grid.shape)
    g = grid_values(grid, {}).as_tensor("torch")
    if g.dtype != torch.float32 or not g.is_contiguous():
        g = g.to(torch.float32).contiguous()
    assert g.numel() == D * H * W, "the majorant grid must hold one value per voxel"
    return g, W, H, D


def _majorant_values(f: VoxelMajorantField) -> tuple[torch.Tensor, int, int, int]:
    """The field's grid values as a contiguous fp32 [D, H, W] tensor and (W, H, D)."""
    return _grid_values_dhw(f.grid)


def voxel_majorant_ptrs(f: VoxelMajorantField, x_ptr: int, y_ptr: int, rows: int) -> None:
    """VoxelMajorantField over `rows` rays (fp32 [rows, 6] at x_ptr) into fp32 [rows, 2] at y_ptr."""
    g, W, H, D = _majorant_values(f)
    _lib.check(_lib.load().rdv_voxel_majorant(C.c_void_p(g.data_ptr()), C.c_int32(W), C.c_int32(H), C.c_int32(D),
                                              C.c_void_p(x_ptr), C.c_int64(rows), C.c_void_p(y_ptr),
                                              C.c_void_p(current_stream_handle())), "VoxelMajorantField")


def voxel_majorant_rows(f: VoxelMajorantField, x) -> RDVObject:
    xt, rows, out = _ray_rows(x, "VoxelMajorantField", 2, ("vmf", id(type(f))))
    with launch_scope():
        voxel_majorant_ptrs(f, xt.data_ptr(), out.device_ptr, rows)
    return out


def _ratio_desc(rt: RatiotrackingTransmittance, seeds, rng_skip: int, W: int, H: int, D: int):
    d = _lib.RatiotrackingDesc()
    for i, v in enumerate(rt.transform.tolist_flat()):
        d.transform[i] = v
    d.density_scale = rt.density_scale
    d.maj_width, d.maj_height, d.maj_depth = W, H, D
    for i, v in enumerate(seeds):
        d.seeds[i] = int(v) & 0xFFFFFFFF
    d.rng_skip = rng_skip
    d.reserved = 0
    return d


def ratiotracking_ptrs(rt: RatiotrackingTransmittance, x_ptr: int, y_ptr: int, rows: int, seeds=None,
                       rng_skip: int = 0) -> None:
    """RatiotrackingTransmittance over `rows` rays (fp32 [rows, 6] at x_ptr) into
    fp32 [rows] at y_ptr; ray i draws from thread i's generator of `seeds`
    (fresh RandomLibrary seeds when None) after skipping rng_skip values."""
    from .types import RandomLibrary
    seeds = RandomLibrary.next_seeds() if seeds is None else seeds
    p, packed = _field_plan(rt.extinction, 3)
    g, W, H, D = _majorant_values(rt.majorant)
    d = _ratio_desc(rt, seeds, rng_skip, W, H, D)
    _lib.check(_lib.load().rdv_ratiotracking_transmittance(
        C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.byref(d), C.c_void_p(g.data_ptr()), C.c_void_p(x_ptr),
        C.c_int64(rows), C.c_void_p(y_ptr), C.c_void_p(current_stream_handle())), "RatiotrackingTransmittance")


def ratiotracking_rows(rt: RatiotrackingTransmittance, x, out: RDVObject | None = None, seeds=None,
                       rng_skip: int = 0) -> RDVObject:
    """RatiotrackingTransmittance over rows x [..., 6] -> [..., 1]."""
    xt, rows, cached = _ray_rows(x, "RatiotrackingTransmittance", 1, ("rtt", id(type(rt))))
    out = cached if out is None else out
    with launch_scope():
        ratiotracking_ptrs(rt, xt.data_ptr(), out.device_ptr, rows, seeds, rng_skip)
    return out


def _vp_desc(vp: VolumeProfile, seeds, rng_skip: int, W: int, H: int, D: int) -> _lib.VolumeProfileDesc:
    if vp.spectral_dim is None:
        raise RuntimeError("Generic arguments could not be deduced from input data. You must explicitly cast.")
    assert 1 <= vp.depth_samples <= _lib.VP_MAX_DEPTH, \
        f"VolumeProfile supports 1..{_lib.VP_MAX_DEPTH} transmittance thresholds"
    assert 1 <= vp.spectral_dim <= _lib.VP_MAX_SPECTRAL, \
        f"VolumeProfile supports a spectral width of 1..{_lib.VP_MAX_SPECTRAL}"
    assert len(vp.light_intensity) == vp.spectral_dim, "light_intensity needs one value per spectral channel"
    d = _lib.VolumeProfileDesc()
    for i, v in enumerate(vp.transform.tolist_flat()):
        d.transform[i] = v
    d.density_scale = vp.density_scale
    d.g = vp.g
    d.step_size = vp.step_size
    for i, v in enumerate(vp.light_direction):
        d.light_direction[i] = v
    for i, v in enumerate(vp.light_intensity):
        d.light_intensity[i] = v
    for i, v in enumerate(vp.transmittance_threshold):
        d.transmittance_threshold[i] = v
    d.depth_samples = vp.depth_samples
    d.spectral_dim = vp.spectral_dim
    d.sample_index = vp.sample_index
    d.environment_samples = vp.environment_samples
    d.maj_width, d.maj_height, d.maj_depth = W, H, D
    for i, v in enumerate(seeds):
        d.seeds[i] = int(v) & 0xFFFFFFFF
    d.rng_skip = rng_skip
    d.reserved = 0
    return d


def _vp_workspace(vp: VolumeProfile, rows: int) -> dict:
    """Per-ray scratch of the two stages (sample positions, environment
    directions and weights, valid flags and the two maps' values), kept on the
    node and reused while the row count is unchanged."""
    es, sd = vp.environment_samples, vp.spectral_dim
    key = (rows, es, sd)
    ws = vp.__dict__.get("_rdv_ws")
    if ws is not None and ws["key"] == key:
        return ws
    dev = device()
    ws = {
        "key": key,
        "spos": torch.empty((max(rows, 1), 3), dtype=torch.float32, device=dev),
        "dirs": torch.empty((max(rows * es, 1), 3), dtype=torch.float32, device=dev),
        "wts": torch.empty((max(rows * es, 1),), dtype=torch.float32, device=dev),
        "valid": torch.empty((max(rows, 1),), dtype=torch.int32, device=dev),
        "albedo": torch.empty((max(rows, 1), sd), dtype=torch.float32, device=dev),
        "env": torch.empty((max(rows * es, 1), sd), dtype=torch.float32, device=dev),
    }
    vp.__dict__["_rdv_ws"] = ws
    return ws


def _map_over(m, x: torch.Tensor, rows: int, out: torch.Tensor) -> tuple[int, int]:
    """(pointer, row stride in floats) of map m's values over the first `rows`
    rows of x: a Constant's one row (stride 0), else m evaluated into `out`."""
    from .maths import Constant
    if isinstance(m, Constant):
        return m._value_ptr(), 0
    if rows > 0:
        _chain.launch_map_rows(m, x.data_ptr(), out.data_ptr(), rows)
    return out.data_ptr(), int(out.shape[1])


def volume_profile_ptrs(vp: VolumeProfile, x_ptr: int, y_ptr: int, rows: int, seeds=None, rng_skip: int = 0) -> None:
    """VolumeProfile over `rows` rays (fp32 [rows, 6] at x_ptr) into fp32
    [rows, OUT] at y_ptr: the ray stage, the scattering-albedo and environment
    maps over its recorded positions and directions, then the finishing stage.
    Ray i draws from thread i's generator of `seeds` (fresh RandomLibrary seeds
    when None) after rng_skip values."""
    from .types import RandomLibrary
    seeds = RandomLibrary.next_seeds() if seeds is None else seeds
    p, packed = _field_plan(vp.extinction, 3)
    g, W, H, D = _majorant_values(vp.majorant)
    d = _vp_desc(vp, seeds, rng_skip, W, H, D)
    ws = _vp_workspace(vp, rows)
    lib = _lib.load()
    stream = C.c_void_p(current_stream_handle())
    tail = (C.c_void_p(x_ptr), C.c_int64(rows), C.c_void_p(y_ptr), C.c_void_p(ws["spos"].data_ptr()),
            C.c_void_p(ws["dirs"].data_ptr()), C.c_void_p(ws["wts"].data_ptr()), C.c_void_p(ws["valid"].data_ptr()),
            stream)
    if isinstance(vp, VolumeProfileDDA):
        dg, dW, dH, dD = _grid_values_dhw(vp.majorant_grid)
        _lib.check(lib.rdv_volume_profile_dda(C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.byref(d),
                                              C.c_void_p(g.data_ptr()), C.c_void_p(dg.data_ptr()), C.c_int32(dW),
                                              C.c_int32(dH), C.c_int32(dD), *tail), "VolumeProfileDDA")
    else:
        _lib.check(lib.rdv_volume_profile(C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.byref(d),
                                          C.c_void_p(g.data_ptr()), *tail), "VolumeProfile")
    a_ptr, a_stride = _map_over(vp.scattering_albedo, ws["spos"], rows, ws["albedo"])
    e_ptr, e_stride = _map_over(vp.environment, ws["dirs"], rows * vp.environment_samples, ws["env"])
    _lib.check(lib.rdv_volume_profile_finish(C.byref(d), C.c_void_p(a_ptr), C.c_int64(a_stride), C.c_void_p(e_ptr),
                                             C.c_int64(e_stride), C.c_void_p(ws["wts"].data_ptr()),
                                             C.c_void_p(ws["valid"].data_ptr()), C.c_int64(rows),
                                             C.c_void_p(y_ptr), stream), "VolumeProfile")


def volume_profile_rows(vp: VolumeProfile, x, out: RDVObject | None = None, seeds=None,
                        rng_skip: int = 0) -> RDVObject:
    """VolumeProfile over rows x [..., 6] -> [..., OUT]."""
    if vp.OUT is None:
        raise RuntimeError("Generic arguments could not be deduced from input data. You must explicitly cast.")
    xt, rows, cached = _ray_rows(x, "VolumeProfile", vp.OUT, ("vp", id(type(vp)), vp.OUT))
    out = cached if out is None else out
    with launch_scope():
        volume_profile_ptrs(vp, xt.data_ptr(), out.device_ptr, rows, seeds, rng_skip)
    return out


def majorant_grid(fine: torch.Tensor, fine_shape, shape, channels: int, aligned: bool, linear: bool,
                  out: torch.Tensor) -> torch.Tensor:
    """MajorantGrid's values: fine [*fine_shape, channels] -> out [*shape, channels]."""
    d = _lib.MajorantGridDesc()
    d.rank = len(shape)
    d.channels = channels
    for i in range(len(shape)):
        d.fine_shape[i] = int(fine_shape[i])
        d.shape[i] = int(shape[i])
    d.aligned = 1 if aligned else 0
    d.linear = 1 if linear else 0
    with launch_scope():
        _lib.check(_lib.load().rdv_majorant_grid(C.byref(d), C.c_void_p(fine.data_ptr()), C.c_void_p(out.data_ptr()),
                                                 C.c_void_p(current_stream_handle())), "MajorantGrid")
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
        if isinstance(m, EmissionAbsorption) and not cam.pixel_jitter:
            return render_ea(cam, m, out)
        # One dispatch's seeds for the camera and the map: the reference's sensor
        # runs both in one thread per cell, whose generator the camera's jitter
        # advances by two draws before the map draws.
        from .types import RandomLibrary
        seeds = RandomLibrary.next_seeds()
        rays = camera_rays(cam, _cached(("sensor-rays",), (*cam.shape, 6)), seeds=seeds)
        if isinstance(m, EmissionAbsorption):
            out = out if out is not None else _cached(("sensor-ea",), (*cam.shape, 3))
            with launch_scope():
                render_ea_rays(m, rays.device_ptr, out.device_ptr, math.prod(cam.shape))
            return out
        if isinstance(m, RaymarchingTransmittance):
            return raymarch_rows(m, rays, out if out is not None else _cached(("sensor-rt",), (*cam.shape, 1)))
        if isinstance(m, VolumeProfile) and m.OUT is not None:
            return volume_profile_rows(m, rays, out if out is not None else _cached(("sensor-vp", m.OUT),
                                                                                     (*cam.shape, m.OUT)),
                                       seeds=seeds, rng_skip=2 if cam.pixel_jitter else 0)
        if isinstance(m, RatiotrackingTransmittance):
            return ratiotracking_rows(m, rays, out if out is not None else _cached(("sensor-rtt",), (*cam.shape, 1)),
                                      seeds=seeds, rng_skip=2 if cam.pixel_jitter else 0)
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


# ------------------------------------------------------ batched evaluation


def _batch_indices(g: Grid, batch) -> tuple[torch.Tensor, tuple, int]:
    """The batch as a contiguous int32 [rows, IN] device tensor, its leading
    shape and row count.  The reference reads the batch as int32 index vectors
    (BatchGridEvaluator's FixArray[INT32, IN]); other integer types are
    converted, floating-point batches raise TypeError."""
    b = wrap(batch)
    t = b.as_tensor("torch")
    if t.dtype.is_floating_point or t.dtype == torch.bool or t.dtype.is_complex:
        raise TypeError(f"grid indices must be integers, got {t.dtype}")
    rank = len(g.shape)
    assert len(t.shape) >= 1 and int(t.shape[-1]) == rank, \
        f"the batch's last dimension ({int(t.shape[-1]) if len(t.shape) else None}) must be the grid's IN ({rank})"
    lead = tuple(int(v) for v in t.shape[:-1])
    rows = math.prod(lead)
    if t.dtype != torch.int32:
        if rows and (int(t.min()) < -(1 << 31) or int(t.max()) >= (1 << 31)):
            raise AssertionError("grid indices must fit in int32")
        t = t.to(torch.int32)
    return t.contiguous().reshape(rows, rank), lead, rows


def _batch_rays(cam: Cameras, idx: torch.Tensor, rows: int, out_ptr: int, seeds) -> None:
    d = camera_desc(cam)
    _lib.check(_lib.load().rdv_cameras_rays_at(C.byref(d), C.c_void_p(_poses(cam).data_ptr()),
                                               C.c_void_p(idx.data_ptr()), C.c_int64(rows),
                                               _seed_array(seeds) if seeds is not None else None,
                                               C.c_void_p(out_ptr), C.c_void_p(current_stream_handle())), "Cameras")


def _node_buffer(node, key: str, shape) -> torch.Tensor:
    """A per-node device buffer reused while its shape is unchanged."""
    shape = tuple(int(s) for s in shape)
    buf = node.__dict__.get(key)
    if buf is None or tuple(buf.shape) != shape:
        buf = torch.empty(shape, dtype=torch.float32, device=device())
        node.__dict__[key] = buf
    return buf


def _batch_values(g: Grid, idx: torch.Tensor, rows: int, out_ptr: int, ctx: dict) -> None:
    """g at the rows index vectors of idx, into fp32 [rows, OUT] at out_ptr."""
    from .grids import _GridNode, grid_values
    if isinstance(g, Cameras):
        seeds = None
        if g.pixel_jitter:
            from .types import RandomLibrary
            seeds = RandomLibrary.next_seeds()
        _batch_rays(g, idx, rows, out_ptr, seeds)
        return
    if isinstance(g, Sensor):
        m = g.map
        if isinstance(g.grid, Cameras):
            cam = g.grid
            # one dispatch's seeds for the camera and the map, as in the full-grid sensor
            from .types import RandomLibrary
            seeds = RandomLibrary.next_seeds()
            rays = _node_buffer(g, "_rdv_batch_rays", (max(rows, 1), 6))
            if rows:
                _batch_rays(cam, idx, rows, rays.data_ptr(), seeds if cam.pixel_jitter else None)
            skip = 2 if cam.pixel_jitter else 0
            if rows == 0:
                return
            if isinstance(m, EmissionAbsorption):
                render_ea_rays(m, rays.data_ptr(), out_ptr, rows)
            elif isinstance(m, RaymarchingTransmittance):
                raymarch_ptrs(m, rays.data_ptr(), out_ptr, rows)
            elif isinstance(m, VolumeProfile):
                volume_profile_ptrs(m, rays.data_ptr(), out_ptr, rows, seeds=seeds, rng_skip=skip)
            elif isinstance(m, RatiotrackingTransmittance):
                ratiotracking_ptrs(m, rays.data_ptr(), out_ptr, rows, seeds=seeds, rng_skip=skip)
            else:
                _chain.launch_map_rows(m, rays.data_ptr(), out_ptr, rows)
            return
        width = g.grid.OUT
        if width is None:
            raise RuntimeError("Generic arguments could not be deduced: the sensor's grid OUT is unknown")
        inner = _node_buffer(g, "_rdv_batch_in", (max(rows, 1), int(width)))
        _batch_values(g.grid, idx, rows, inner.data_ptr(), ctx)
        if rows == 0:
            return
        if isinstance(m, EmissionAbsorption):
            render_ea_rays(m, inner.data_ptr(), out_ptr, rows)
        else:
            _chain.launch_map_rows(m, inner.data_ptr(), out_ptr, rows)
        return
    # a grid whose values this build materialises (TensorGrid, barriers,
    # convolutions, resampling, majorant grids, ...): its values, gathered
    v = grid_values(g, ctx) if isinstance(g, _GridNode) else evaluate_grid(g)
    vt = v.as_tensor("torch")
    if vt.dtype != torch.float32 or not vt.is_contiguous():
        vt = vt.to(torch.float32).contiguous()
    rank = len(g.shape)
    width = int(vt.numel() // max(1, math.prod(g.shape)))
    shape = (C.c_int64 * rank)(*[int(s) for s in g.shape])
    _lib.check(_lib.load().rdv_grid_gather(C.c_void_p(vt.data_ptr()), C.c_int32(rank), shape, C.c_int32(width),
                                           C.c_void_p(idx.data_ptr()), C.c_int64(rows), C.c_void_p(out_ptr),
                                           C.c_void_p(current_stream_handle())), "Grid batch")


def evaluate_grid_batch(g: Grid, batch) -> RDVObject:
    """g at a batch of index vectors [..., IN] -> [..., OUT] fp32, in an output
    buffer cached per grid class and batch shape (maths:104-119)."""
    if g.OUT is None:
        raise RuntimeError("Generic arguments could not be deduced: the grid's OUT is unknown")
    idx, lead, rows = _batch_indices(g, batch)
    out = _cached(("batch", id(type(g)), int(g.OUT)), (*lead, int(g.OUT)))
    with launch_scope():
        _batch_values(g, idx, rows, out.device_ptr, {})
    return out
