"""Camera, transmittance and volume-rendering nodes of the rdv API.

  Cameras                    reference domain/rendering.py:10-42 (Grid[3, 6])
  RaymarchingTransmittance   reference domain/volumes.py:124-141 (Map[6, 1])
  RatiotrackingTransmittance reference domain/volumes.py:144-190 (Map[6, 1])
  VoxelMajorantField         reference domain/volumes.py:191-211 (Map[6, 2])
  VolumeProfile              reference domain/volumes.py:503-550 (Map[6, DS + 3 SD + 4])
  EmissionAbsorption         build-defined (Map[6, 3]): the MLP-in-the-loop
                             renderer of the benchmark configuration
  ExtinctionTrait, MajorantTrait, RatiotrackingTransmittanceTrait,
  RaymarchingTransmittanceTrait, ScatteringAlbedoTrait, EnvironmentTrait,
  EnvironmentSamplerTrait    reference domain/volumes.py:7-120: the keyword
                             constructors that hold, cast and bind a volume
                             node's component maps
Grids compose with maps (`Cameras(...) >> RaymarchingTransmittance(m)`) into a
Sensor; calling the sensor renders every pixel on the GPU.
"""
from __future__ import annotations

import math

import torch

from .core import RDVObject, wrap
from .maths import Grid, Map
from .types import Code, Generic, Generics, _MatBase, generic_value, mat4x3


class Cameras(Grid[3, 6]):
    """Pinhole cameras: cell (c, y, x) -> (origin, unit direction) of the ray
    through pixel (x, y) of camera c (reference: rendering.py:10-42,
    shaders/rendering/cameras.h).  poses: [num_cameras, 9] = origin | target | up.
    aspect_ratio defaults to width / height and fov (vertical, radians) to pi / 4.
    jitter: each evaluation places every ray at a uniform random point of its
    pixel (two random() draws of the cell's thread, RandomLibrary) instead of
    the centre."""

    IN = 3
    OUT = 6

    def __init__(self, width: int, height: int, poses, aspect_ratio: float | None = None, fov: float | None = None,
                 jitter: bool = False) -> None:
        if aspect_ratio is None:
            aspect_ratio = width / height
        if fov is None:
            fov = math.pi / 4
        if not isinstance(poses, RDVObject):
            poses = wrap(torch.as_tensor(poses, dtype=torch.float32))
        assert poses.shape[1] == 9, "poses must be a [num_cameras, 9] tensor (ori | target | up)"
        super().__init__([poses.shape[0], height, width])
        self.poses = poses
        self.width = int(width)
        self.height = int(height)
        self.aspect_ratio = float(aspect_ratio)
        self.fov = float(fov)
        self.pixel_jitter = 1 if jitter else 0


def _as_mat4x3(t) -> mat4x3:
    """A transform given as a mat4x3, a 4x3 nested list / tensor (rows are the
    columns: three linear columns, then the translation) or 12 floats in that
    column-major order."""
    if isinstance(t, _MatBase):
        return mat4x3(t)
    vals = [float(v) for v in torch.as_tensor(t, dtype=torch.float64).reshape(-1)]
    assert len(vals) == 12, "transform must be a mat4x3 (12 values)"
    return mat4x3(*vals)


# ------------------------------------------------------------------ traits


def _bound(node, name: str):
    """The value bound to generic `name` on node: by its class, its own
    attribute, or a match() made earlier in the same constructor."""
    v = generic_value(node, name)
    if v is None:
        v = node.__dict__.get("_rdv_pending", {}).get(name)
    return v


class ExtinctionTrait(Code, Generic[Generics.EXTINCTION]):
    """Holds `extinction`, cast to a Map[3, 1]; binds EXTINCTION to its type
    (reference: volumes.py:7-19)."""

    def __init__(self, *, extinction, **kwargs) -> None:
        extinction = extinction.cast(Map[3, 1])
        self.match(Generics.EXTINCTION, type(extinction))
        self.extinction = extinction
        super().__init__(**kwargs)


class EnvironmentSamplerTrait(Code, Generic[Generics.ENVIRONMENT_SAMPLER, Generics.SPECTRAL_DIM]):
    """Holds `environment_sampler`, cast to a Map[6, SPECTRAL_DIM + 4]; binds
    SPECTRAL_DIM from its width when still open (reference: volumes.py:22-41)."""

    def __init__(self, *, environment_sampler, **kwargs) -> None:
        spectral_dim = _bound(self, "SPECTRAL_DIM")
        if spectral_dim is None and environment_sampler.OUT is not None:
            spectral_dim = environment_sampler.OUT - 4
        environment_sampler = environment_sampler.cast(Map[6, None if spectral_dim is None else spectral_dim + 4])
        self.match(Generics.ENVIRONMENT_SAMPLER, type(environment_sampler))
        self.match(Generics.SPECTRAL_DIM, spectral_dim)
        self.environment_sampler = environment_sampler
        super().__init__(**kwargs)


class EnvironmentTrait(Code, Generic[Generics.ENVIRONMENT, Generics.SPECTRAL_DIM]):
    """Holds `environment`, cast to a Map[3, SPECTRAL_DIM]; binds SPECTRAL_DIM
    from its width when still open (reference: volumes.py:44-63)."""

    def __init__(self, *, environment, **kwargs) -> None:
        spectral_dim = _bound(self, "SPECTRAL_DIM")
        if spectral_dim is None:
            spectral_dim = environment.OUT
        environment = environment.cast(Map[3, spectral_dim])
        self.match(Generics.ENVIRONMENT, type(environment))
        self.match(Generics.SPECTRAL_DIM, spectral_dim)
        self.environment = environment
        super().__init__(**kwargs)


class ScatteringAlbedoTrait(Code, Generic[Generics.SCATTERING_ALBEDO, Generics.SPECTRAL_DIM]):
    """Holds `scattering_albedo`, cast to a Map[3, SPECTRAL_DIM]; binds
    SPECTRAL_DIM from its width when still open (reference: volumes.py:66-85)."""

    def __init__(self, *, scattering_albedo, **kwargs) -> None:
        spectral_dim = _bound(self, "SPECTRAL_DIM")
        if spectral_dim is None:
            spectral_dim = scattering_albedo.OUT
        scattering_albedo = scattering_albedo.cast(Map[3, spectral_dim])
        self.match(Generics.SCATTERING_ALBEDO, type(scattering_albedo))
        self.match(Generics.SPECTRAL_DIM, spectral_dim)
        self.scattering_albedo = scattering_albedo
        super().__init__(**kwargs)


class MajorantTrait(Code, Generic[Generics.MAJORANT]):
    """Holds `majorant`: a VoxelMajorantField, or a Grid[3, 1] wrapped as one,
    cast to a Map[6, 2] (reference: volumes.py:88-102)."""

    def __init__(self, *, majorant, **kwargs) -> None:
        majorant = _as_majorant_field(majorant).cast(Map[6, 2])
        self.match(Generics.MAJORANT, type(majorant))
        self.majorant = majorant
        super().__init__(**kwargs)


class RatiotrackingTransmittanceTrait(ExtinctionTrait, MajorantTrait):
    """Extinction and majorant: what ratio tracking needs (reference:
    volumes.py:105-111)."""


class RaymarchingTransmittanceTrait(ExtinctionTrait):
    """Extinction: what a fixed-step raymarch needs (reference: volumes.py:114-120)."""


class RaymarchingTransmittance(Map[6, 1], RaymarchingTransmittanceTrait):
    """T(x, w) along a ray through the box [-1,1]^3 of the object space given by
    `transform` (mat4x3, column-major: three linear columns, then the translation),
    marched with fixed steps: tau += extinction(x) * density_scale * step_size,
    0 once tau > 16, exp(-tau) at the end; 1 when the ray misses
    (reference: volumes.py:124-141, shaders/volumes/raymarching_transmittance.h).
    extinction: a Map[3, 1]: a chain of LinearFast (fp16) and Linear (exact
    fp32) layers from 3 inputs (raw or frequency-encoded) to 1 output, or a
    Constant; evaluated on the matrix cores for 32 march steps at a time
    (chains with a Linear layer: widths up to 64)."""

    IN = 6
    OUT = 1

    def __init__(self, extinction: Map, transform=None, step_size: float = 0.002, density_scale: float = 1.0) -> None:
        super().__init__(extinction=extinction)  # TypeError for any other width (volumes.py:16)
        self.transform = mat4x3(1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0) \
            if transform is None else _as_mat4x3(transform)
        self.step_size = float(step_size)
        self.density_scale = float(density_scale)

    def _evaluate_rows(self, x) -> RDVObject:
        from . import _render
        return _render.raymarch_rows(self, x)

    def _launch_rows(self, x_ptr: int, y_ptr: int, rows: int) -> None:
        from . import _render
        _render.raymarch_ptrs(self, x_ptr, y_ptr, rows)


class VoxelMajorantField(Map[6, 2]):
    """(x, w) -> (majorant, distance): the value of the voxel of `grid` (a
    Grid[3, 1] over the box [-1,1]^3, shape [D, H, W]) that holds x, and the
    distance along w to that voxel's exit (reference: volumes.py:191-211,
    shaders/volumes/voxel_majorant_field.h).  Every voxel value must bound the
    extinction over its voxel, or ratio tracking is biased."""

    IN = 6
    OUT = 2

    def __init__(self, grid) -> None:
        grid = grid.cast(Grid[3, 1])
        assert len(grid.shape) == 3, "VoxelMajorantField needs a 3-D grid"
        self.grid = grid

    def _grid_values(self) -> RDVObject:
        from .grids import grid_values
        return grid_values(self.grid, {})

    def _evaluate_rows(self, x) -> RDVObject:
        from . import _render
        return _render.voxel_majorant_rows(self, x)

    def _launch_rows(self, x_ptr: int, y_ptr: int, rows: int) -> None:
        from . import _render
        _render.voxel_majorant_ptrs(self, x_ptr, y_ptr, rows)


def _as_majorant_field(majorant) -> VoxelMajorantField:
    """A majorant field as given, or a bare Grid[3, 1] wrapped as one
    (reference: volumes.py:235-254)."""
    if isinstance(majorant, VoxelMajorantField):
        return majorant
    if isinstance(majorant, Grid) and majorant.OUT == 1:
        return VoxelMajorantField(majorant)
    raise NotImplementedError("majorant must be a VoxelMajorantField or a Grid[3, 1]")


class RatiotrackingTransmittance(Map[6, 1], RatiotrackingTransmittanceTrait):
    """T(x, w) along a ray through the box [-1,1]^3 of the object space given by
    `transform`, estimated by ratio tracking against a voxel majorant field:
    free flights of -log(1 - random()) / (majorant * density_scale) capped at
    the voxel exit, T *= 1 - extinction(x) / majorant at each collision,
    Russian roulette below T = 0.05, at most 1024 steps; 1 when the ray misses
    (reference: volumes.py:144-190, shaders/volumes/ratiotracking_transmittance.h,
    ratiotracking_transmittance_trait.h).  An unbiased, noisy estimate: each
    evaluation draws fresh random seeds (RandomLibrary).
    extinction: a Map[3, 1] (a chain of LinearFast / Linear layers from 3 inputs
    to 1 output, widths up to 64 with a Linear layer, or a Constant);
    majorant: a VoxelMajorantField or a Grid[3, 1] (wrapped as one)."""

    IN = 6
    OUT = 1

    def __init__(self, extinction: Map, majorant, transform=None, density_scale: float = 1.0) -> None:
        super().__init__(extinction=extinction, majorant=majorant)
        self.transform = mat4x3(1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0) \
            if transform is None else _as_mat4x3(transform)
        self.density_scale = float(density_scale)

    def _evaluate_rows(self, x) -> RDVObject:
        from . import _render
        return _render.ratiotracking_rows(self, x)

    def _launch_rows(self, x_ptr: int, y_ptr: int, rows: int) -> None:
        from . import _render
        _render.ratiotracking_ptrs(self, x_ptr, y_ptr, rows)


class VolumeProfile(Map, RatiotrackingTransmittanceTrait, RaymarchingTransmittanceTrait, ScatteringAlbedoTrait,
                    EnvironmentTrait, Generic[Generics.DEPTH_SAMPLES]):
    """Per-ray features of a participating medium for a learned renderer
    (reference: volumes.py:503-550, shaders/volumes/volume_profile.h:1-167).
    For a ray (x, w) [6] in the object space of `transform` (the box [-1,1]^3),
    OUT = DS + 3 SD + 4 values (DS = len(transmittance_threshold), SD = the
    spectral width of scattering_albedo / environment):
      [0, DS)            re-encoded depths where tau crosses each threshold's
                         expected crossing value (1 / (0.1 + t_0), then
                         1 / (1 + 10 sqrt(t_i - t_{i-1})))
      DS                 0.2 log(1 + tau)
      DS + 1             S * T of the light ray (raymarched, step_size)
      DS + 2 + [0, SD)   environment next-event estimate: mean over
                         environment_samples Henyey-Greenstein directions of
                         S * T (ratio-tracked) * environment(direction)
      DS + 2 + SD + [0, SD)   1 / (1 - log(1 - albedo)) at the sample position
      DS + 2 + 2 SD      g
      DS + 3 + 2 SD + [0, SD)  light_intensity
      OUT - 1            S = 1 - exp(-tau)
    (everything but S is 0 where no depth was reached; all 0 for a miss).
    extinction: a Map[3, 1] (a chain of LinearFast / Linear layers from 3 inputs
    to 1 output, widths up to 64 with a Linear layer, or a Constant);
    majorant: a VoxelMajorantField or a Grid[3, 1]; scattering_albedo and
    environment: Map[3, SD] (Constant maps or any map this package evaluates
    over rows).  Random draws: ray i uses thread i's generator of a fresh
    dispatch (RandomLibrary).  nee_near_distance is kept for the interface; the
    reference's active shader does not read it."""

    IN = 6

    def __init__(self, extinction: Map, majorant, environment: Map, scattering_albedo: Map,
                 transmittance_threshold: list, density_scale: float = 1.0, transform=None,
                 light_direction=(0.0, 1.0, 0.0), light_intensity=None, g: float = 0.0, step_size: float = 0.001,
                 environment_samples: int = 4, sample_index: int = 0, nee_near_distance: float = 0.05) -> None:
        # the traits in the reference's order (volumes.py:7-120): extinction, majorant,
        # scattering albedo (fixes SPECTRAL_DIM when the map's width is known), environment
        super().__init__(extinction=extinction, majorant=majorant, environment=environment,
                         scattering_albedo=scattering_albedo)
        spectral_dim = _bound(self, "SPECTRAL_DIM")
        depth_samples = len(transmittance_threshold)
        self.match(Generics.DEPTH_SAMPLES, depth_samples)
        self.spectral_dim = None if spectral_dim is None else int(spectral_dim)
        self.depth_samples = depth_samples
        self.OUT = None if spectral_dim is None else 4 + spectral_dim * 3 + depth_samples
        self.transform = mat4x3(1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0) \
            if transform is None else _as_mat4x3(transform)
        self.light_direction = tuple(float(v) for v in light_direction)
        assert len(self.light_direction) == 3, "light_direction must have 3 components"
        if spectral_dim is not None:
            self.light_intensity = [1.0] * spectral_dim if light_intensity is None else \
                [float(v) for v in light_intensity]
        self.density_scale = float(density_scale)
        self.g = float(g)
        self.step_size = float(step_size)
        self.environment_samples = int(environment_samples)
        self.sample_index = int(sample_index)
        self.transmittance_threshold = [float(v) for v in transmittance_threshold]
        self.nee_near_distance = float(nee_near_distance)

    def _evaluate_rows(self, x) -> RDVObject:
        from . import _render
        return _render.volume_profile_rows(self, x)

    def _launch_rows(self, x_ptr: int, y_ptr: int, rows: int) -> None:
        from . import _render
        _render.volume_profile_ptrs(self, x_ptr, y_ptr, rows)


class VolumeProfileDDA(VolumeProfile):
    """VolumeProfile whose primary ray walks `majorant_grid` cell by cell
    (reference: volumes.py:560-603, shaders/volumes/volume_profile_dda.h:1-208).
    The tau and depth marches use an Amanatides-Woo DDA over majorant_grid, a
    Grid[3, 1] of shape [D, H, W] over the box (e.g. a MajorantGrid's output),
    instead of trimming the ray's ends with `majorant`. A cell whose value is
    > 0 is marched in fixed steps from where the walk entered it up to its exit.
    Cells whose value is not > 0 are skipped whole. At most 4096 cells are
    walked, stopping at the box exit or on leaving the grid. `majorant` (the
    VoxelMajorantField) still serves the environment rays' ratio tracking, and
    the outputs are VolumeProfile's."""

    def __init__(self, extinction: Map, majorant, majorant_grid, environment: Map, scattering_albedo: Map,
                 transmittance_threshold: list, density_scale: float = 1.0, transform=None,
                 light_direction=(0.0, 1.0, 0.0), light_intensity=None, g: float = 0.0, step_size: float = 0.001,
                 environment_samples: int = 4, sample_index: int = 0, nee_near_distance: float = 0.05) -> None:
        super().__init__(extinction=extinction, majorant=majorant, environment=environment,
                         scattering_albedo=scattering_albedo, transmittance_threshold=transmittance_threshold,
                         density_scale=density_scale, transform=transform, light_direction=light_direction,
                         light_intensity=light_intensity, g=g, step_size=step_size,
                         environment_samples=environment_samples, sample_index=sample_index,
                         nee_near_distance=nee_near_distance)
        majorant_grid = majorant_grid.cast(Grid[3, 1])
        assert len(majorant_grid.shape) == 3, "VolumeProfileDDA needs a 3-D majorant_grid"
        self.majorant_grid = majorant_grid


class EmissionAbsorption(Map[6, 3]):
    """Build-defined volume renderer (no reference counterpart): along each ray
    (origin, direction) through [-1,1]^3, `samples` points t_i = t0 + (i + 1/2) dt
    are fed through `field` (Map[3, 4]: density logit, RGB logits; any
    LinearFast chain with a raw head), with
    sigma = softplus, c = sigmoid, and composited front to back:
    alpha_i = 1 - exp(-sigma_i dt), T_i = prod_{j<i} (1 - alpha_j),
    C = sum_i T_i alpha_i c_i (0 for rays that miss)."""

    IN = 6
    OUT = 3

    def __init__(self, field: Map, samples: int = 128) -> None:
        field = field.cast(Map[3, 4])  # TypeError for any other width
        assert samples >= 32 and samples % 32 == 0, "samples must be a positive multiple of 32"
        self.field = field
        self.samples = int(samples)

    def _evaluate_rows(self, x) -> RDVObject:
        from . import _render
        x = wrap(x)
        if x.scalar_type != torch.float32:
            raise TypeError(f"Map input must be float32, got {x.scalar_type}")
        assert x.shape[-1] == 6, "EmissionAbsorption expects rows of 6 values (origin, direction)"
        xt = x.as_tensor("torch").contiguous()
        rows = xt.numel() // 6
        out = _render._cached(("ea-rows", id(type(self))), (*x.shape[:-1], 3))
        from .core import launch_scope
        with launch_scope():
            _render.render_ea_rays(self, xt.data_ptr(), out.device_ptr, rows)
        return out

    def _launch_rows(self, x_ptr: int, y_ptr: int, rows: int) -> None:
        from . import _render
        _render.render_ea_rays(self, x_ptr, y_ptr, rows)
