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


def test_volume_traits_are_public_and_bind_their_maps():
    for name in ["ExtinctionTrait", "MajorantTrait", "RatiotrackingTransmittanceTrait",
                 "RaymarchingTransmittanceTrait", "ScatteringAlbedoTrait", "EnvironmentTrait",
                 "EnvironmentSamplerTrait", "MemoryLocation"]:
        assert hasattr(rdv, name), name
    ext = _chain([3, 64, 64, 1])
    rt = rdv.RaymarchingTransmittance(ext)
    assert isinstance(rt, rdv.RaymarchingTransmittanceTrait) and isinstance(rt, rdv.ExtinctionTrait)
    assert rdv.Generics.EXTINCTION(rt) is type(ext) and rt.extinction is ext
    maj = rdv.TensorGrid(torch.ones(2, 2, 2, 1))
    rtt = rdv.RatiotrackingTransmittance(ext, maj)
    assert isinstance(rtt, rdv.RatiotrackingTransmittanceTrait) and isinstance(rtt, rdv.MajorantTrait)
    assert isinstance(rtt.majorant, rdv.VoxelMajorantField) and rdv.Generics.MAJORANT(rtt) is rdv.VoxelMajorantField
    vp = rdv.VolumeProfile(ext, maj, rdv.Constant(torch.ones(1, 2)), rdv.Constant(torch.ones(1, 2)), [0.5, 0.2, 0.1])
    for t in (rdv.RatiotrackingTransmittanceTrait, rdv.RaymarchingTransmittanceTrait, rdv.ScatteringAlbedoTrait,
              rdv.EnvironmentTrait):
        assert isinstance(vp, t)
    assert rdv.Generics.SPECTRAL_DIM(vp) == 2 and rdv.Generics.DEPTH_SAMPLES(vp) == 3 and vp.OUT == 4 + 6 + 3
    with pytest.raises(TypeError):  # the environment's width disagrees with the albedo's
        rdv.VolumeProfile(ext, maj, rdv.Constant(torch.ones(1, 3)), rdv.Constant(torch.ones(1, 2)), [0.5])
    with pytest.raises(TypeError):  # not a Map[3, 1]
        rdv.RatiotrackingTransmittance(_chain([3, 64, 2]), maj)

    class Custom(rdv.Map[6, 1], rdv.RaymarchingTransmittanceTrait):
        def __init__(self, extinction):
            super().__init__(extinction=extinction)

    c = Custom(ext)
    assert isinstance(c, rdv.ExtinctionTrait) and c.extinction is ext
    with pytest.raises(TypeError):
        rdv.ExtinctionTrait(extinction=_chain([3, 8, 2]))


def test_constant_is_the_first_row():
    data = torch.tensor([[1.0, 2.0], [3.0, 4.0]])
    c = rdv.Constant(data)
    assert c.OUT == 2
    ptr = c._value_ptr()
    assert ptr == c.buf_.device_ptr  # the buffer's first OUT floats, not its last row


def test_ensure_on_rdv_returns_the_callers_backend_in_owned_memory():
    import numpy as np
    a = np.arange(6, dtype=np.float32).reshape(2, 3)
    b = rdv.ensure_on_rdv(a)
    assert isinstance(b, np.ndarray) and b.shape == (2, 3) and (b == a).all()
    assert b.__array_interface__["data"][0] != a.__array_interface__["data"][0]
    assert rdv.is_on_rdv(b) and not rdv.is_on_rdv(a) and rdv.is_on_rdv(b[1:])
    assert rdv.ensure_on_rdv(b) is b  # already the library's: unchanged
    t = torch.arange(5.0)
    u = rdv.ensure_on_rdv(t)
    assert isinstance(u, torch.Tensor) and u.data_ptr() != t.data_ptr() and torch.equal(u, t)
    assert rdv.is_on_rdv(u) and not rdv.is_on_rdv(t) and rdv.ensure_on_rdv(u) is u
    v = rdv.ensure_on_rdv(a, backend="torch")
    assert isinstance(v, torch.Tensor) and v.shape == (2, 3) and rdv.is_on_rdv(v)
    with pytest.raises(ValueError):
        rdv.ensure_on_rdv(a, backend="numpy", location=rdv.MemoryLocation.DEVICE)
    with pytest.raises(TypeError):
        rdv.ensure_on_rdv([1.0, 2.0])
    del u
    import gc
    gc.collect()
    assert not rdv.is_on_rdv(t)


def test_grid_batch_rejects_bad_indices_before_launch():
    cam = rdv.Cameras(8, 6, torch.tensor([[0.0, 0.0, -3.5, 0.0, 0.0, 0.0, 0.0, 1.0, 0.0]]))
    with pytest.raises(TypeError):
        cam(torch.zeros(4, 3))
    with pytest.raises(AssertionError):
        cam(torch.zeros(4, 2, dtype=torch.int32))
    with pytest.raises(AssertionError):
        cam(torch.zeros(4, 3, dtype=torch.int32), torch.zeros(4, 3, dtype=torch.int32))
