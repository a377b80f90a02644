"""The C ABI library loads and exports every symbol include/*.h declares;
host-only entry points (validation, sizes) behave (CPU only, no launches)."""
import ctypes as C
import glob
import os
import re

import pytest

from rdv_project_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(rdv_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return sorted(names)


def test_header_declares_functions():
    names = _declared_functions()
    assert "rdv_mlp_forward" in names and "rdv_last_error" in names


@pytest.mark.parametrize("name", _declared_functions())
def test_library_exports_declared_symbol(name):
    lib = _lib.load()
    assert hasattr(lib, name), f"{name} declared in include/ but not exported by librdv_hip.so"


def test_binding_covers_header():
    assert set(_lib.exported_symbols()) == set(_declared_functions())


def _desc(dims, acts=None, precs=None, enc=_lib.ENC_NONE, octaves=0, in_features=None):
    d = _lib.MlpDesc()
    d.n_layers = len(dims) - 1
    d.in_features = in_features if in_features is not None else dims[0]
    d.encoding = enc
    d.enc_octaves = octaves
    for i, v in enumerate(dims):
        d.dims[i] = v
    for i in range(d.n_layers):
        d.act[i] = (acts or [_lib.ACT_RELU] * d.n_layers)[i]
        d.prec[i] = (precs or [_lib.PREC_F16] * d.n_layers)[i]
    return d


def test_validate_accepts_benchmark_chains():
    lib = _lib.load()
    assert lib.rdv_mlp_validate(C.byref(_desc([3, 64, 64, 64, 64, 4]))) == 0
    assert lib.rdv_mlp_validate(C.byref(_desc([48, 64, 64, 64, 4], enc=_lib.ENC_FREQ, octaves=6,
                                              in_features=3))) == 0


@pytest.mark.parametrize("dims,kw,fragment", [
    ([3, 64, 4], dict(in_features=5), "must match"),
    ([3, 0, 4], {}, "outside"),
    ([3, 300, 4], {}, "outside"),
    ([30, 64, 4], dict(enc=_lib.ENC_FREQ, octaves=6, in_features=3), "encoded width"),
])
def test_validate_rejects(dims, kw, fragment):
    lib = _lib.load()
    rc = lib.rdv_mlp_validate(C.byref(_desc(dims, **kw)))
    assert rc == _lib.RDV_ERR_INVALID
    assert fragment in _lib.last_error()


def test_validate_rejects_layer_count():
    lib = _lib.load()
    d = _desc([3, 4])
    d.n_layers = 0
    assert lib.rdv_mlp_validate(C.byref(d)) == _lib.RDV_ERR_INVALID
    d.n_layers = 17
    assert lib.rdv_mlp_validate(C.byref(d)) == _lib.RDV_ERR_INVALID


def test_packed_bytes_layout():
    lib = _lib.load()
    # 3->64->4: frag 2x1 + 1x4 tiles of 1 KiB, 256-aligned biases, fp32 copies
    n = lib.rdv_mlp_packed_bytes(C.byref(_desc([3, 64, 4])))
    sections = [2 * 1 * 1024, 1 * 4 * 1024,  # fp16 A fragments: MT x KC x 1 KiB
                64 * 4, 32 * 4,              # padded fp32 biases
                64 * 3 * 4, 4 * 64 * 4,      # fp32 weight copies
                64 * 4, 4 * 4]               # fp32 bias copies
    off = 256  # header (magic, per-layer bias flags)
    for s in sections:  # every section starts 256-byte aligned
        off = (off + s + 255) // 256 * 256
    assert n == off
    # exact fp32 layers hold fp32 fragments for v_mfma_f32_32x32x2f32: MT x KB (32-row K blocks) x 4 KiB
    n32 = lib.rdv_mlp_packed_bytes(C.byref(_desc([3, 64, 4], precs=[0, 0])))
    sections[0:2] = [2 * 1 * 4 * 1024, 1 * 2 * 4 * 1024]
    off = 256
    for s in sections:
        off = (off + s + 255) // 256 * 256
    assert n32 == off
    # the unpacked entry needs no workspace where a compile-time kernel serves the chain
    assert lib.rdv_mlp_unpacked_workspace_bytes(C.byref(_desc([3, 64, 64, 64, 64, 4], acts=[1, 1, 1, 1, 0]))) == 0
    assert lib.rdv_mlp_unpacked_workspace_bytes(C.byref(_desc([3, 64, 4]))) == n
    assert lib.rdv_mlp_unpacked_workspace_bytes(C.byref(_desc([3, 64, 4], precs=[0, 0]))) == n32


def test_kernel_selection_names():
    lib = _lib.load()
    assert lib.rdv_mlp_kernel_name(C.byref(_desc([3, 64, 64, 64, 64, 4], acts=[1, 1, 1, 1, 0]))) \
        .decode().startswith("mlp_fused_f16<raw3,64x4,4>")
    assert lib.rdv_mlp_kernel_name(C.byref(
        _desc([48, 64, 64, 64, 4], acts=[1, 1, 1, 0], enc=_lib.ENC_FREQ, octaves=6, in_features=3))) \
        .decode() == "mlp_fused_f16<freq3x6,64x3,4>"
    # fp32 layers go to the vector-ALU chain kernels (register rows up to 64 wide), unlisted
    # LinearFast shapes to the generic kernel
    assert lib.rdv_mlp_kernel_name(C.byref(_desc([3, 64, 4], precs=[0, 0]))).decode() == "mlp_chain_f32_reg_kernel"
    assert lib.rdv_mlp_kernel_name(C.byref(_desc([3, 128, 4], precs=[0, 0]))).decode() == "mlp_chain_f32_kernel"
    assert lib.rdv_mlp_kernel_name(C.byref(_desc([5, 37, 19]))).decode() == "mlp_generic_f16<2,lds>"
    assert lib.rdv_mlp_kernel_name(C.byref(_desc([3, 256, 256, 4]))).decode() == "mlp_generic_f16<8,global>"


def _conv(**kw):
    d = _lib.ConvDesc()
    vals = dict(batch=1, H=256, W=256, cin=64, cout=64, in_layout=_lib.LAYOUT_CHW, in_dtype=_lib.DTYPE_F16,
                out_layout=_lib.LAYOUT_CHW, out_dtype=_lib.DTYPE_F16, relu=1)
    vals.update(kw)
    for k, v in vals.items():
        setattr(d, k, v)
    return d


def test_winograd_validate_accepts_benchmark_and_reference_shapes():
    lib = _lib.load()
    assert lib.rdv_winograd3x3_validate(_conv()) == 0
    assert lib.rdv_winograd3x3_validate(_conv(H=16, W=16, cin=48, cout=48, in_layout=_lib.LAYOUT_HWC,
                                              in_dtype=_lib.DTYPE_F32, out_layout=_lib.LAYOUT_HWC,
                                              out_dtype=_lib.DTYPE_F32, relu=0)) == 0
    assert lib.rdv_winograd3x3_validate(_conv(H=2, W=2, cin=1, cout=16)) == 0


@pytest.mark.parametrize("kw,fragment", [
    (dict(H=255), "even"),
    (dict(W=0), "even"),
    (dict(cin=65), "in_channels"),
    (dict(cin=0), "in_channels"),
    (dict(cout=40), "out_channels"),
    (dict(cout=2048), "out_channels"),
    (dict(batch=0), "batch"),
    (dict(in_layout=7), "layout"),
    (dict(out_dtype=5), "element type"),
    (dict(H=8192, W=8192), "2^31"),
])
def test_winograd_validate_rejects(kw, fragment):
    lib = _lib.load()
    assert lib.rdv_winograd3x3_validate(_conv(**kw)) == _lib.RDV_ERR_INVALID
    assert fragment in _lib.last_error()


def test_winograd_weight_bytes():
    lib = _lib.load()
    # [16 positions][ceil(cin/32)][cout/16][64 lanes][8] fp16
    assert lib.rdv_winograd3x3_weight_bytes(64, 64) == 16 * 2 * 4 * 64 * 8 * 2
    assert lib.rdv_winograd3x3_weight_bytes(5, 16) == 16 * 1 * 1 * 64 * 8 * 2
    assert lib.rdv_winograd3x3_weight_bytes(64, 40) == _lib.RDV_ERR_INVALID


def _lin(rows=4096, inf=128, outf=128, prec=_lib.PREC_F16, wkind=_lib.WKIND_F32, relu=0):
    d = _lib.LinearOpDesc()
    d.rows, d.in_features, d.out_features, d.precision, d.wkind, d.relu, d.reserved = rows, inf, outf, prec, wkind, relu, 0
    return d


def test_linear_op_validate_accepts_reference_shapes():
    lib = _lib.load()
    for d in (_lin(), _lin(rows=4, inf=8, outf=8, prec=_lib.PREC_F32), _lin(inf=4096, outf=1000),
              _lin(inf=32, outf=16, wkind=_lib.WKIND_F16), _lin(rows=64, inf=64, outf=96, wkind=_lib.WKIND_F16_TILED16),
              _lin(rows=0)):
        assert lib.rdv_linear_op_validate(C.byref(d)) == 0, _lib.last_error()


@pytest.mark.parametrize("kw,fragment", [
    (dict(inf=12), "in_features"),
    (dict(inf=0), "in_features"),
    (dict(outf=6), "out_features"),
    (dict(rows=-1), "rows"),
    (dict(prec=7), "precision"),
    (dict(wkind=9), "weight kind"),
    (dict(prec=_lib.PREC_F32, wkind=_lib.WKIND_F16), "fp32 weight"),
    (dict(inf=24, wkind=_lib.WKIND_F16_TILED16), "tiled"),
])
def test_linear_op_validate_rejects(kw, fragment):
    lib = _lib.load()
    assert lib.rdv_linear_op_validate(C.byref(_lin(**kw))) == _lib.RDV_ERR_INVALID
    assert fragment in _lib.last_error()


def test_linear_op_host_errors_need_no_device():
    lib = _lib.load()
    # invalid descriptor, NULL and misaligned pointers are refused before any HIP call
    assert lib.rdv_linear_op(C.byref(_lin(inf=12)), None, None, None, None, None) == _lib.RDV_ERR_INVALID
    assert lib.rdv_linear_op(C.byref(_lin()), None, None, None, None, None) == _lib.RDV_ERR_INVALID
    assert "NULL" in _lib.last_error()
    assert lib.rdv_linear_op(C.byref(_lin()), 0x1004, 0x2000, 0x3000, 0x4000, None) == _lib.RDV_ERR_INVALID
    assert "aligned" in _lib.last_error()
    assert lib.rdv_linear_op(C.byref(_lin(rows=0)), None, None, None, None, None) == 0
    assert lib.rdv_relu_op(None, None, -1, None) == _lib.RDV_ERR_INVALID
    assert lib.rdv_relu_op(None, None, 0, None) == 0
    assert lib.rdv_relu_op(0x1008, 0x2000, 16, None) == _lib.RDV_ERR_INVALID


def _vp(**kw):
    d = _lib.VolumeProfileDesc()
    for i, v in enumerate([1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0]):
        d.transform[i] = v
    d.density_scale, d.g, d.step_size = 1.0, 0.0, 0.001
    d.light_direction[1] = 1.0
    d.depth_samples, d.spectral_dim, d.sample_index, d.environment_samples = 3, 3, 0, 4
    d.maj_width = d.maj_height = d.maj_depth = 8
    d.rng_skip, d.reserved = 0, 0
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def _ext_desc():
    d = _lib.MlpDesc()
    d.n_layers, d.in_features, d.encoding, d.enc_octaves = 2, 3, _lib.ENC_NONE, 0
    d.dims[0], d.dims[1], d.dims[2] = 3, 16, 1
    d.act[0], d.act[1] = _lib.ACT_RELU, _lib.ACT_NONE
    d.prec[0] = d.prec[1] = _lib.PREC_F16
    return d


@pytest.mark.parametrize("kw,fragment", [
    (dict(depth_samples=0), "depth_samples"),
    (dict(depth_samples=17), "depth_samples"),
    (dict(spectral_dim=0), "spectral_dim"),
    (dict(spectral_dim=9), "spectral_dim"),
    (dict(sample_index=3), "sample_index"),
    (dict(environment_samples=-1), "environment_samples"),
    (dict(step_size=0.0), "step_size"),
    (dict(density_scale=-1.0), "density_scale"),
    (dict(maj_depth=0), "majorant grid"),
    (dict(rng_skip=-2), "rng_skip"),
    (dict(reserved=1), "reserved"),
])
def test_volume_profile_rejects_before_any_launch(kw, fragment):
    lib = _lib.load()
    d = _vp(**kw)
    rc = lib.rdv_volume_profile(C.byref(_ext_desc()), 0x1000, C.byref(d), 0x2000, 0x3000, 64, 0x4000, 0x5000,
                                0x6000, 0x7000, 0x8000, None)
    assert rc == _lib.RDV_ERR_INVALID and fragment in _lib.last_error()
    rc = lib.rdv_volume_profile_finish(C.byref(d), 0x1000, 3, 0x2000, 3, 0x3000, 0x4000, 64, 0x5000, None)
    assert rc == _lib.RDV_ERR_INVALID and fragment in _lib.last_error()


@pytest.mark.parametrize("w,h,dd,grid,fragment", [
    (0, 4, 4, 0x9000, "grid dimensions"),
    (4, 4097, 4, 0x9000, "grid dimensions"),
    (4, 4, 4, None, "NULL"),
])
def test_volume_profile_dda_rejects_before_any_launch(w, h, dd, grid, fragment):
    lib = _lib.load()
    d = _vp()
    rc = lib.rdv_volume_profile_dda(C.byref(_ext_desc()), 0x1000, C.byref(d), 0x2000, grid, w, h, dd, 0x3000, 64,
                                    0x4000, 0x5000, 0x6000, 0x7000, 0x8000, None)
    assert rc == _lib.RDV_ERR_INVALID and fragment in _lib.last_error()
    # the VolumeProfile descriptor checks come first, as for rdv_volume_profile
    rc = lib.rdv_volume_profile_dda(C.byref(_ext_desc()), 0x1000, C.byref(_vp(depth_samples=0)), 0x2000, 0x9000,
                                    4, 4, 4, 0x3000, 64, 0x4000, 0x5000, 0x6000, 0x7000, 0x8000, None)
    assert rc == _lib.RDV_ERR_INVALID and "depth_samples" in _lib.last_error()
    assert lib.rdv_volume_profile_dda(C.byref(_ext_desc()), None, C.byref(d), None, None, 4, 4, 4, None, 0, None,
                                      None, None, None, None, None) == 0


def test_volume_profile_host_errors_need_no_device():
    lib = _lib.load()
    d = _vp()
    assert lib.rdv_volume_profile(C.byref(_ext_desc()), None, C.byref(d), None, None, 0, None, None, None, None,
                                  None, None) == 0
    assert lib.rdv_volume_profile(C.byref(_ext_desc()), None, C.byref(d), None, None, 16, None, None, None, None,
                                  None, None) == _lib.RDV_ERR_INVALID
    assert "NULL" in _lib.last_error()
    assert lib.rdv_volume_profile_finish(C.byref(d), 0x1000, -1, 0x2000, 3, 0x3000, 0x4000, 8, 0x5000,
                                         None) == _lib.RDV_ERR_INVALID
    assert lib.rdv_broadcast_rows(None, 0, 4, None, None) == _lib.RDV_ERR_INVALID
    assert lib.rdv_broadcast_rows(None, 3, 0, None, None) == 0
