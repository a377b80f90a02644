"""The reference's public call patterns on the hot path keep working with
`import rdv_project_amd as rdv` (construction and type checks only; nothing
here launches a kernel, so it runs without a GPU)."""
import math

import pytest
import torch

import rdv_project_amd as rdv


def _chain(dims, f16=True):
    g = torch.Generator().manual_seed(0)
    m = None
    for i in range(len(dims) - 1):
        lin = rdv.linear(torch.randn(dims[i + 1], dims[i], generator=g), torch.zeros(dims[i + 1]), f16=f16)
        m = lin if m is None else m >> rdv.relu >> lin
    return m


def test_curated_names_import():
    for name in ["linear", "Linear", "LinearFast", "relu", "ReLU", "LinearTensorOp", "LinearTensorOpSmall",
                 "LinearTensorOpSimple", "LinearTensorOpFast", "LinearTensorOpMine", "Conv2DTensorOp",
                 "Conv2DTensorOpFast", "Conv2DTensorOpSimple", "Conv2DTensorOpSimple3x3", "Conv2DTensorOpWindow3x3",
                 "Conv2DTensorOpWinograd3x3", "Downsample2xTensorOp", "Upsample2xTensorOp", "ConcatTensorOp",
                 "Cameras", "RaymarchingTransmittance", "RatiotrackingTransmittance", "VoxelMajorantField",
                 "VolumeProfile", "VolumeProfileDDA", "MajorantGrid", "TensorGrid", "wrap", "dispatch", "profiling", "profiling_submit_times",
                 "reset_submit_times", "Map", "Grid", "X", "Generics", "Generic", "Main", "Component", "Struct",
                 "Library", "Single", "Array", "Pointer", "Buffer", "FixArray", "Deferred", "deferreds",
                 "RDVObject", "ensure_on_rdv", "is_on_rdv", "MathLibrary", "RandomLibrary", "GridLibrary",
                 "CooperativeLibrary", "DeferredLibrary", "mat2", "mat3", "mat4", "mat3x4", "mat4x3", "vec2",
                 "vec3", "vec4", "ivec2", "ivec3", "ivec4", "uvec2", "uvec3", "uvec4", "bvec2", "bvec3", "bvec4",
                 "MapEvaluator", "GridEvaluator", "TensorOpEvaluator", "TensorOperation"]:
        assert hasattr(rdv, name), name


def test_map_subscript_and_isinstance():
    m = _chain([3, 64, 64, 1])
    assert isinstance(m, rdv.Map) and isinstance(m, rdv.Map[3, 1]) and not isinstance(m, rdv.Map[3, 4])
    assert rdv.Generics.IN(m) == 3 and rdv.Generics.OUT(m) == 1
    assert m.cast(rdv.Map[3, 1]) is m
    with pytest.raises(TypeError):
        m.cast(rdv.Map[6, 1])
    assert rdv.Map[3, 1] is rdv.Map[rdv.Generics.IN: 3, rdv.Generics.OUT: 1]
    assert isinstance(rdv.relu, rdv.Map) and rdv.relu.IN is None  # generic until composed


def test_raymarching_transmittance_with_mat4x3_transform():
    m = _chain([3, 64, 64, 64, 1])
    M = rdv.mat4x3(1.5, 0.0, 0.0, 0.0, 1.5, 0.0, 0.0, 0.0, 1.5, 0.2, -0.1, 0.3)
    rt = rdv.RaymarchingTransmittance(m, transform=M, step_size=0.01, density_scale=2.0)
    assert isinstance(rt, rdv.Map[6, 1]) and rt.transform == M and rt.transform[3] == [0.2, -0.1, 0.3]
    rt2 = rdv.RaymarchingTransmittance(extinction=m, transform=[[1.5, 0, 0], [0, 1.5, 0], [0, 0, 1.5], [0.2, -0.1, 0.3]],
                                       step_size=0.01, density_scale=2.0)
    assert rt2.transform == M
    assert rdv.RaymarchingTransmittance(m).transform == rdv.mat4x3(1, 0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 0)
    with pytest.raises(TypeError):
        rdv.RaymarchingTransmittance(_chain([3, 64, 4]))   # not a Map[3, 1]


def test_camera_grid_composition():
    poses = torch.tensor([[0.0, 0.0, -3.5, 0.0, 0.0, 0.0, 0.0, 1.0, 0.0]])
    cam = rdv.Cameras(8, 6, poses)
    assert isinstance(cam, rdv.Grid[3, 6]) and cam.shape == [1, 6, 8]
    assert cam.fov == pytest.approx(math.pi / 4) and cam.aspect_ratio == pytest.approx(8 / 6)
    s = cam >> rdv.RaymarchingTransmittance(_chain([3, 64, 64, 64, 1]))
    assert isinstance(s, rdv.Sensor) and s.OUT == 1 and s.shape == [1, 6, 8]


def test_deferred_bindings():
    t = torch.zeros(3)
    d = rdv.Deferred("density")
    with pytest.raises(RuntimeError):
        d.resolve()
    with rdv.deferreds(density=t):
        assert d.resolve() is t
    with pytest.raises(RuntimeError):
        d.resolve()
    assert rdv.Deferred(obj=t).resolve() is t


def test_vectors_and_matrices():
    v = rdv.vec3(1, 2, 3)
    assert (v.x, v.y, v.z) == (1.0, 2.0, 3.0) and list(v) == [1.0, 2.0, 3.0]
    assert rdv.vec4(0.5).w == 0.5
    assert rdv.mat3() == rdv.mat3(1.0)                  # identity
    m = rdv.mat4x3(*range(12))
    assert m[1] == [3.0, 4.0, 5.0] and len(m) == 4    # column-major: 4 columns of 3
    with pytest.raises(ValueError):
        rdv.mat4x3(1, 2, 3)


def test_dispatch_rejects_non_main():
    with pytest.raises(TypeError):
        rdv.dispatch(_chain([3, 4]), 32)
