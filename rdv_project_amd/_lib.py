"""ctypes binding of librdv_hip.so (the C ABI declared in include/rdv_hip.h).

The library is built in-tree by rdv_project_amd/build.py.  Nothing here falls
back to a CPU implementation: if the shared library is missing, or no GPU is
visible, every compute call raises.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

_PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG_DIR, "librdv_hip.so")

RDV_OK = 0
RDV_ERR_INVALID = -1
RDV_ERR_UNSUPPORTED = -2
RDV_ERR_HIP = -3
RDV_ERR_WORKSPACE = -4

MLP_MAX_LAYERS = 16
MLP_MAX_WIDTH = 256
TRAIN_STATIC_SCRATCH_BYTES = 64 << 20  # RDV_TRAIN_STATIC_SCRATCH_BYTES

ACT_NONE, ACT_RELU, ACT_SOFTPLUS, ACT_SIGMOID, ACT_DENSITY_RGB = 0, 1, 2, 3, 4
PREC_F32, PREC_F16 = 0, 1
ENC_NONE, ENC_FREQ = 0, 1
LAYOUT_HWC, LAYOUT_CHW = 0, 1
DTYPE_F32, DTYPE_F16 = 0, 1
WLAYOUT_RSCK, WLAYOUT_KCRS = 0, 1
WKIND_F32, WKIND_F16, WKIND_F16_TILED16 = 0, 1, 2


class MlpDesc(C.Structure):
    """Mirror of rdv_mlp_desc."""
    _fields_ = [
        ("n_layers", C.c_int32),
        ("in_features", C.c_int32),
        ("encoding", C.c_int32),
        ("enc_octaves", C.c_int32),
        ("dims", C.c_int32 * (MLP_MAX_LAYERS + 1)),
        ("act", C.c_int32 * MLP_MAX_LAYERS),
        ("prec", C.c_int32 * MLP_MAX_LAYERS),
    ]


class ConvDesc(C.Structure):
    """Mirror of rdv_conv_desc."""
    _fields_ = [
        ("batch", C.c_int32),
        ("H", C.c_int32),
        ("W", C.c_int32),
        ("cin", C.c_int32),
        ("cout", C.c_int32),
        ("in_layout", C.c_int32),
        ("in_dtype", C.c_int32),
        ("out_layout", C.c_int32),
        ("out_dtype", C.c_int32),
        ("relu", C.c_int32),
    ]


class CameraDesc(C.Structure):
    """Mirror of rdv_camera_desc."""
    _fields_ = [
        ("n_cams", C.c_int32),
        ("width", C.c_int32),
        ("height", C.c_int32),
        ("aspect_ratio", C.c_float),
        ("fov", C.c_float),
    ]


class LinearOpDesc(C.Structure):
    """Mirror of rdv_linear_op_desc."""
    _fields_ = [
        ("rows", C.c_int64),
        ("in_features", C.c_int32),
        ("out_features", C.c_int32),
        ("precision", C.c_int32),
        ("wkind", C.c_int32),
        ("relu", C.c_int32),
        ("reserved", C.c_int32),
    ]


class Conv2dDesc(C.Structure):
    """Mirror of rdv_conv2d_desc."""
    _fields_ = [
        ("H", C.c_int32),
        ("W", C.c_int32),
        ("cin", C.c_int32),
        ("cout", C.c_int32),
        ("kh", C.c_int32),
        ("kw", C.c_int32),
        ("precision", C.c_int32),
        ("w_layout", C.c_int32),
        ("relu", C.c_int32),
        ("reserved", C.c_int32),
    ]


class RatiotrackingDesc(C.Structure):
    """Mirror of rdv_ratiotracking_desc."""
    _fields_ = [
        ("transform", C.c_float * 12),
        ("density_scale", C.c_float),
        ("maj_width", C.c_int32),
        ("maj_height", C.c_int32),
        ("maj_depth", C.c_int32),
        ("seeds", C.c_uint32 * 4),
        ("rng_skip", C.c_int32),
        ("reserved", C.c_int32),
    ]


VP_MAX_DEPTH = 16
VP_MAX_SPECTRAL = 8


class VolumeProfileDesc(C.Structure):
    """Mirror of rdv_volume_profile_desc."""
    _fields_ = [
        ("transform", C.c_float * 12),
        ("density_scale", C.c_float),
        ("g", C.c_float),
        ("step_size", C.c_float),
        ("light_direction", C.c_float * 3),
        ("light_intensity", C.c_float * VP_MAX_SPECTRAL),
        ("transmittance_threshold", C.c_float * VP_MAX_DEPTH),
        ("depth_samples", C.c_int32),
        ("spectral_dim", C.c_int32),
        ("sample_index", C.c_int32),
        ("environment_samples", C.c_int32),
        ("maj_width", C.c_int32),
        ("maj_height", C.c_int32),
        ("maj_depth", C.c_int32),
        ("seeds", C.c_uint32 * 4),
        ("rng_skip", C.c_int32),
        ("reserved", C.c_int32),
    ]


class MajorantGridDesc(C.Structure):
    """Mirror of rdv_majorant_grid_desc."""
    _fields_ = [
        ("rank", C.c_int32),
        ("channels", C.c_int32),
        ("fine_shape", C.c_int32 * 4),
        ("shape", C.c_int32 * 4),
        ("aligned", C.c_int32),
        ("linear", C.c_int32),
    ]


GRID_MAX_RANK = 8


class RDVError(RuntimeError):
    """A HIP runtime failure reported by the library."""


_SIGNATURES = {
    "rdv_last_error": (C.c_char_p, []),
    "rdv_version": (C.c_int, []),
    "rdv_device_cu_count": (C.c_int, []),
    "rdv_mlp_validate": (C.c_int, [C.POINTER(MlpDesc)]),
    "rdv_mlp_packed_bytes": (C.c_int64, [C.POINTER(MlpDesc)]),
    "rdv_mlp_pack": (C.c_int, [C.POINTER(MlpDesc), C.POINTER(C.c_void_p), C.POINTER(C.c_void_p), C.c_void_p,
                               C.c_void_p]),
    "rdv_mlp_forward": (C.c_int, [C.POINTER(MlpDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    "rdv_mlp_unpacked_workspace_bytes": (C.c_int64, [C.POINTER(MlpDesc)]),
    "rdv_mlp_forward_unpacked": (C.c_int, [C.POINTER(MlpDesc), C.POINTER(C.c_void_p), C.POINTER(C.c_void_p),
                                           C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_int64, C.c_void_p]),
    "rdv_mlp_forward_f16_all": (C.c_int, [C.POINTER(MlpDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                          C.c_void_p]),
    "rdv_mlp_kernel_name": (C.c_char_p, [C.POINTER(MlpDesc)]),
    "rdv_mlp_train_workspace_bytes": (C.c_int64, [C.POINTER(MlpDesc), C.c_int64]),
    "rdv_mlp_train_step": (C.c_int, [C.POINTER(MlpDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p,
                                     C.c_int64, C.c_void_p, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p),
                                     C.c_void_p]),
    "rdv_mlp_train_step_static": (C.c_int, [C.POINTER(MlpDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64,
                                            C.c_void_p, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p), C.c_void_p]),
    "rdv_cameras_rays": (C.c_int, [C.POINTER(CameraDesc), C.c_void_p, C.c_void_p, C.c_void_p]),
    "rdv_cameras_rays_jittered": (C.c_int, [C.POINTER(CameraDesc), C.c_void_p, C.POINTER(C.c_uint32), C.c_void_p,
                                            C.c_void_p]),
    "rdv_cameras_rays_at": (C.c_int, [C.POINTER(CameraDesc), C.c_void_p, C.c_void_p, C.c_int64,
                                      C.POINTER(C.c_uint32), C.c_void_p, C.c_void_p]),
    "rdv_grid_gather": (C.c_int, [C.c_void_p, C.c_int32, C.POINTER(C.c_int64), C.c_int32, C.c_void_p, C.c_int64,
                                  C.c_void_p, C.c_void_p]),
    "rdv_random_uniform": (C.c_int, [C.POINTER(C.c_uint32), C.c_int64, C.c_int32, C.c_void_p, C.c_void_p]),
    "rdv_ratiotracking_transmittance": (C.c_int, [C.POINTER(MlpDesc), C.c_void_p, C.POINTER(RatiotrackingDesc),
                                                  C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p]),
    "rdv_voxel_majorant": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_int64, C.c_void_p,
                                     C.c_void_p]),
    "rdv_majorant_grid": (C.c_int, [C.POINTER(MajorantGridDesc), C.c_void_p, C.c_void_p, C.c_void_p]),
    "rdv_volume_profile": (C.c_int, [C.POINTER(MlpDesc), C.c_void_p, C.POINTER(VolumeProfileDesc), C.c_void_p,
                                     C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_void_p, C.c_void_p]),
    "rdv_volume_profile_dda": (C.c_int, [C.POINTER(MlpDesc), C.c_void_p, C.POINTER(VolumeProfileDesc), C.c_void_p,
                                         C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_int64,
                                         C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "rdv_volume_profile_finish": (C.c_int, [C.POINTER(VolumeProfileDesc), C.c_void_p, C.c_int64, C.c_void_p,
                                            C.c_int64, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p]),
    "rdv_broadcast_rows": (C.c_int, [C.c_void_p, C.c_int32, C.c_int64, C.c_void_p, C.c_void_p]),
    "rdv_render_emission_absorption": (C.c_int, [C.POINTER(CameraDesc), C.c_void_p, C.POINTER(MlpDesc), C.c_void_p,
                                                 C.c_int32, C.c_void_p, C.c_void_p]),
    "rdv_render_emission_absorption_rays": (C.c_int, [C.POINTER(MlpDesc), C.c_void_p, C.c_void_p, C.c_int64,
                                                      C.c_int32, C.c_void_p, C.c_void_p]),
    "rdv_composite": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_int32, C.c_void_p, C.c_void_p]),
    "rdv_raymarch_transmittance": (C.c_int, [C.POINTER(MlpDesc), C.c_void_p, C.c_void_p, C.c_int64,
                                             C.POINTER(C.c_float), C.c_float, C.c_float, C.c_void_p, C.c_void_p]),
    "rdv_linear_op_validate": (C.c_int, [C.POINTER(LinearOpDesc)]),
    "rdv_linear_op": (C.c_int, [C.POINTER(LinearOpDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                C.c_void_p]),
    "rdv_relu_op": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p]),
    "rdv_conv2d_validate": (C.c_int, [C.POINTER(Conv2dDesc)]),
    "rdv_conv2d": (C.c_int, [C.POINTER(Conv2dDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "rdv_downsample2x": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int32, C.c_void_p, C.c_void_p]),
    "rdv_upsample2x": (C.c_int, [C.c_void_p, C.c_int64, C.c_int64, C.c_int32, C.c_void_p, C.c_void_p]),
    "rdv_concat_channels": (C.c_int, [C.c_void_p, C.c_int32, C.c_void_p, C.c_int32, C.c_int64, C.c_void_p,
                                      C.c_void_p]),
    "rdv_winograd3x3_validate": (C.c_int, [C.POINTER(ConvDesc)]),
    "rdv_winograd3x3_weight_bytes": (C.c_int64, [C.c_int32, C.c_int32]),
    "rdv_winograd3x3_transform_weight": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                                   C.c_void_p, C.c_void_p]),
    "rdv_winograd3x3_forward": (C.c_int, [C.POINTER(ConvDesc), C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                          C.c_void_p]),
}

_lib = None
_lock = threading.Lock()


def exported_symbols() -> list[str]:
    """Every symbol this binding expects the library to export."""
    return list(_SIGNATURES)


def load(path: str | None = None):
    """Loads (once) and returns the ctypes handle; raises if the library is missing."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"{p} not found: the HIP extension is not built (run `python -m rdv_project_amd.build`). "
                "There is no CPU fallback.")
        lib = C.CDLL(p)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def last_error() -> str:
    return load().rdv_last_error().decode()


def check(rc: int, what: str = "") -> None:
    """Maps an rdv_status to the exception type the reference raises for it."""
    if rc == RDV_OK:
        return
    msg = last_error()
    prefix = f"{what}: " if what else ""
    if rc == RDV_ERR_INVALID:
        raise AssertionError(prefix + msg)
    if rc == RDV_ERR_UNSUPPORTED:
        raise NotImplementedError(prefix + msg)
    raise RDVError(prefix + f"[{rc}] {msg}")


def void_ptr_array(ptrs) -> C.Array:
    arr = (C.c_void_p * max(1, len(ptrs)))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr
