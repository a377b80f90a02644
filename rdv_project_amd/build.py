"""Builds librdv_hip.so (all HIP kernels + the C ABI) for gfx950, in-tree.

Every source is compiled by hipcc to an object under rdv_project_amd/_build/
(in parallel), then linked into rdv_project_amd/librdv_hip.so.  The flag
`-Xclang -target-feature -Xclang -packed-fp32-ops` keeps the compiler from
forming packed fp32 instructions.

    python -m rdv_project_amd.build      # or: from rdv_project_amd.build import build; build()
"""
from __future__ import annotations

import concurrent.futures as _cf
import os
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "librdv_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)

# Longest compiles first: the pool starts them in this order.
SOURCES = [
    "mlp_generic8.hip",
    "mlp_generic8g.hip",
    "render.hip",
    "render_field8_march.hip",
    "render_field8_ratio.hip",
    "render_field8_ea.hip",
    "volume_profile.hip",
    "volume_profile8.hip",
    "volume_profile_dda.hip",
    "volume_profile_dda8.hip",
    "mlp_generic.hip",
    "train.hip",
    "winograd.hip",
    "conv_op.hip",
    "mlp_fused.hip",
    "linear_op.hip",
    "capi.cpp",
    "mlp_pack.hip",
    "mlp_f32.hip",
    "tensor_data.hip",
    "grid_batch.hip",
]

ARCH = os.environ.get("RDV_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = os.path.join(rocm, "bin", "hipcc")
    return cand if os.path.exists(cand) else "hipcc"


def _compile(src: str, extra: list[str]) -> str:
    obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{res.stdout}\n{_filter(res.stderr)}")
    return obj


def _filter(text: str) -> str:
    # hipcc's host pass does not know the packed-fp32 feature name; that warning is noise.
    return "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l)


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> str:
    """Compiles every source and links the shared library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    extra = list(extra_flags or [])
    jobs = min(len(SOURCES), max(1, min(8, os.cpu_count() or 1)))
    with _cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{_filter(res.stderr)}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
