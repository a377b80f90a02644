#!/usr/bin/env python
"""Benchmark of the rdv small-network hot path on one MI355X.

Headline (the JSON line's `value`): configuration C2 of BASELINE.json — the
encoded coordinate MLP, 2^20 points, FREQ(6 octaves) 39 -> pad 48 -> 64 -> 64 ->
64 -> 4, fp16 matrix cores with fp32 accumulation, one fused kernel per call.
A step is one call over the 2^20 points with inputs already resident in HBM
(buffer sets rotate so the 256 MB MALL does not serve them).

    python bench.py [--steps K] [--warmup W] [--gpus 1]

Prints ONE JSON line.  One clock throughout: `value`, `ms_per_step` and
`roofline` all come from HIP events recorded on the stream the kernels run on,
around exactly the K timed steps (the wall-clock time of the same region, with
its synchronisations, is reported beside them as `wall_ms_per_step`).
`cpu_baseline` times this repo's torch-CPU restatement (oracle/torch_cpu.py) on
the host cores, C1 in full and bounded samples of C2-C5.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "fused-MLP Mpoints/s (w64, 2^20 pts) + % fp16 MFMA peak; Winograd conv TFLOP/s"
PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
PEAK_FP32_TFLOPS = 157.3   # MI355X fp32 (vector and matrix)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
C2_FLOP_PER_POINT = 2 * (48 * 64 + 64 * 64 + 64 * 64 + 64 * 4)  # 23,040 (declared padded shapes)
C1_FLOP_PER_POINT = 2 * (3 * 64 + 3 * 64 * 64 + 64 * 4)          # 25,472
ROTATE = 12
# C3: direct-equivalent work 2 H W CIN COUT 9 (the convention for reporting
# convolution TFLOP/s); Winograd-domain MFMA work 2 * 16 * tiles * CIN * COUT;
# algorithmic HBM bytes: fp16 x + fp16 y + packed fp16 U.
C3_DIRECT_FLOP = 2 * 256 * 256 * 64 * 64 * 9                     # 4.832 GFLOP
C3_WINO_FLOP = 2 * 16 * (128 * 128) * 64 * 64                     # 2.147 GFLOP
C3_BYTES = 2 * 64 * 256 * 256 * 2 + 16 * 2 * 4 * 64 * 8 * 2       # 16,908,288 B
C3_ROTATE = 24  # 24 x (8 + 8) MiB of x / y: more than the 256 MB MALL
# C4: per-sample work of the 3 -> 64 -> 64 -> 64 -> 4 field; compositing kernel
# traffic per ray: 128 samples x 16 B read, 4 B dt read, 12 B colour written.
C4_FLOP_PER_SAMPLE = 2 * (3 * 64 + 64 * 64 + 64 * 64 + 64 * 4)   # 17,280
C4_COMPOSITE_BYTES_PER_RAY = 128 * 16 + 4 + 12
# C5: forward 2 (32 128 + 7 128^2 + 128 16), dW the same, dX of layers 2..9
C5_FLOP_PER_POINT = 241664 + 241664 + 233472                        # 716,800
# Runtime-shaped matrix-core MLP (no compile-time instance): 2^20 points, 64 -> 128 -> 128 -> 128 -> 16
GEN_DIMS = [64, 128, 128, 128, 16]
GEN_FLOP_PER_POINT = 2 * sum(GEN_DIMS[i] * GEN_DIMS[i + 1] for i in range(len(GEN_DIMS) - 1))  # 86,016


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _mlp_setup(x_cpu, layers, acts, enc=None, rotate=ROTATE, f16=True):
    """Builds the rdv chain (LinearFast layers, or exact-fp32 Linear ones with
    f16=False), packs it, and returns (desc, packed, rotating x/y sets)."""
    import torch
    import rdv_project_amd as rdv
    from rdv_project_amd import _chain

    m = enc
    for (w, b), a in zip(layers, acts):
        lin = rdv.linear(w.cuda(), b.cuda(), f16=f16)
        m = lin if m is None else m >> lin
        if a == "relu":
            m = m >> rdv.relu
    p = _chain.plan_chain(m, x_cpu.shape[1])
    packed = _chain.packed_params(m, p)
    xd = x_cpu.cuda()
    xs = [xd] + [xd.clone() for _ in range(rotate - 1)]
    ys = [torch.empty(x_cpu.shape[0], p.out_features, device="cuda") for _ in range(rotate)]
    return m, p, packed, xs, ys


PREWARM_S = 0.5  # seconds of untimed launches before the warm-up steps


def bench_volume_profile(steps, warmup):
    """VolumeProfile over the C4 camera's 512 x 512 rays: the ratio-tracking leg's extinction (3 -> 64 -> 64 -> 64
    -> 1 softplus, seed 11) and 8^3 majorant, density_scale 4, thresholds (0.9, 0.5, 0.1), step_size 0.004, g 0.3,
    4 environment samples, constant RGB environment and albedo (the two maps cost nothing); both stages timed.
    Then VolumeProfileDDA on the same rays, its walked grid the same 8^3 MajorantGrid."""
    import torch
    import rdv_project_amd as rdv
    from rdv_project_amd import _chain, _lib, _render
    from rdv_project_amd import workloads as WL
    from rdv_project_amd.types import RandomLibrary
    lib = _lib.load()
    layers = WL.kaiming_uniform_f16([(64, 3), (64, 64), (64, 64), (1, 64)], seed=11)
    ext = None
    for i, (w, b) in enumerate(layers):
        lin = rdv.linear(w.cuda(), b.cuda(), f16=True)
        ext = lin if ext is None else ext >> lin
        ext = ext >> (rdv.relu if i + 1 < len(layers) else rdv.softplus)
    c = (torch.arange(64, dtype=torch.float32) + 0.5) / 64 * 2 - 1
    zz, yy, xx = torch.meshgrid(c, c, c, indexing="ij")
    lattice = torch.stack([xx, yy, zz], -1).reshape(-1, 3).cuda()
    dens = ext(rdv.wrap(lattice)).as_tensor("torch").reshape(64, 64, 64, 1) * 1.3 + 1e-3
    mg = rdv.MajorantGrid(rdv.TensorGrid(dens.clone()), [8, 8, 8])
    majv = mg().as_tensor("torch").contiguous().clone()
    vp = rdv.VolumeProfile(ext, mg, rdv.Constant([1.0, 0.9, 0.8]), rdv.Constant([0.6, 0.7, 0.8]), [0.9, 0.5, 0.1],
                           density_scale=4.0, g=0.3, step_size=0.004, environment_samples=4)
    p = _chain.plan_chain(ext, 3)
    packed = _chain.packed_params(ext, p)
    rays = rdv.Cameras(WL.C4_WIDTH, WL.C4_HEIGHT, WL.c4_pose().cuda())().as_tensor("torch").reshape(-1, 6).clone()
    n = rays.shape[0]
    out = torch.empty(n, vp.OUT, device="cuda")
    RandomLibrary.seed(0)
    d = _render._vp_desc(vp, RandomLibrary.next_seeds(), 0, 8, 8, 8)
    ws = _render._vp_workspace(vp, n)
    env_v, alb_v = vp.environment._value_ptr(), vp.scattering_albedo._value_ptr()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def launch(i):
        d.seeds[0] = 256 + i
        rc = lib.rdv_volume_profile(C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.byref(d),
                                    C.c_void_p(majv.data_ptr()), C.c_void_p(rays.data_ptr()), C.c_int64(n),
                                    C.c_void_p(out.data_ptr()), C.c_void_p(ws["spos"].data_ptr()),
                                    C.c_void_p(ws["dirs"].data_ptr()), C.c_void_p(ws["wts"].data_ptr()),
                                    C.c_void_p(ws["valid"].data_ptr()), stream)
        if rc == 0:
            rc = lib.rdv_volume_profile_finish(C.byref(d), C.c_void_p(alb_v), C.c_int64(0), C.c_void_p(env_v),
                                               C.c_int64(0), C.c_void_p(ws["wts"].data_ptr()),
                                               C.c_void_p(ws["valid"].data_ptr()), C.c_int64(n),
                                               C.c_void_p(out.data_ptr()), stream)
        if rc != 0:
            _lib.check(rc, "volume profile")

    wall, ev = _time_launches(launch, steps, warmup, prewarm_s=0.0)
    valid = float(ws["valid"][:n].float().mean())
    mean_s = float(out[:, -1].double().mean())

    def launch_dda(i):  # VolumeProfileDDA: the primary ray walks the same 8^3 MajorantGrid cell by cell
        d.seeds[0] = 256 + i
        rc = lib.rdv_volume_profile_dda(C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.byref(d),
                                        C.c_void_p(majv.data_ptr()), C.c_void_p(majv.data_ptr()), C.c_int32(8),
                                        C.c_int32(8), C.c_int32(8), C.c_void_p(rays.data_ptr()), C.c_int64(n),
                                        C.c_void_p(out.data_ptr()), C.c_void_p(ws["spos"].data_ptr()),
                                        C.c_void_p(ws["dirs"].data_ptr()), C.c_void_p(ws["wts"].data_ptr()),
                                        C.c_void_p(ws["valid"].data_ptr()), stream)
        if rc == 0:
            rc = lib.rdv_volume_profile_finish(C.byref(d), C.c_void_p(alb_v), C.c_int64(0), C.c_void_p(env_v),
                                               C.c_int64(0), C.c_void_p(ws["wts"].data_ptr()),
                                               C.c_void_p(ws["valid"].data_ptr()), C.c_int64(n),
                                               C.c_void_p(out.data_ptr()), stream)
        if rc != 0:
            _lib.check(rc, "volume profile DDA")

    _, ev_dda = _time_launches(launch_dda, steps, warmup, prewarm_s=0.0)
    return {
        "workload": "VolumeProfile over 512x512 C4 camera rays: extinction 3->64->64->64->1 softplus (fp16 MFMA, "
                    "seed 11), 8^3 voxel majorant, density_scale 4, thresholds (0.9, 0.5, 0.1), step 0.004, g 0.3, "
                    "4 environment samples, constant RGB environment and albedo",
        "kernels": "volume_profile64_kernel (the chain compiled for this shape, 64 rays per wave) + "
                   "volume_profile_finish_kernel",
        "ms_per_call": round(ev, 3),
        "Mrays_per_s": round(n / (ev * 1e-3) / 1e6, 2),
        "valid_fraction": round(valid, 4),
        "mean_S": round(mean_s, 4),
        "dda": {"ms_per_call": round(ev_dda, 3), "Mrays_per_s": round(n / (ev_dda * 1e-3) / 1e6, 2),
                "valid_fraction": round(float(ws["valid"][:n].float().mean()), 4),
                "mean_S": round(float(out[:, -1].double().mean()), 4),
                "variant": "VolumeProfileDDA, majorant_grid = the same 8^3 MajorantGrid"},
        "bound": "per-ray state machine (two fixed-step marches, the light ray's march, four ratio-tracked "
                 "environment rays); one chain evaluation per step for the 64 rays of a wave, as two staggered "
                 "32-point tiles",
    }


def _time_launches(launch, steps: int, warmup: int, prewarm_s: float | None = None):
    """Returns (wall ms per step, event ms per step) for `steps` back-to-back
    launches.  Before the `warmup` steps the same launches run, untimed, for
    `prewarm_s` seconds: the GPU takes longer than a few hundred short launches
    to reach its steady-state clock (the first 40 ms of C2 launches run ~7%
    slower than the rest), and the benchmark reports the steady state."""
    import torch
    t_end = time.perf_counter() + (PREWARM_S if prewarm_s is None else prewarm_s)
    i = 0
    while time.perf_counter() < t_end:
        for _ in range(64):
            launch(i)
            i += 1
        torch.cuda.synchronize()
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        launch(i)
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ev = start.elapsed_time(end) / steps
    return wall, ev


def bench_mlp(x_cpu, layers, acts, enc, steps, warmup, rotate=ROTATE, f16=True):
    import torch
    from rdv_project_amd import _lib
    lib = _lib.load()
    m, p, packed, xs, ys = _mlp_setup(x_cpu, layers, acts, enc, rotate, f16)
    n = x_cpu.shape[0]
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    dptr = C.byref(p.desc)
    pk = C.c_void_p(packed.data_ptr())
    xp = [C.c_void_p(t.data_ptr()) for t in xs]
    yp = [C.c_void_p(t.data_ptr()) for t in ys]
    nn = C.c_int64(n)
    fwd = lib.rdv_mlp_forward

    def launch(i):
        k = i % rotate
        rc = fwd(dptr, pk, xp[k], yp[k], nn, stream)
        if rc != 0:
            _lib.check(rc, "mlp forward")

    wall, ev = _time_launches(launch, steps, warmup)
    name = lib.rdv_mlp_kernel_name(dptr).decode()
    return wall, ev, name


def bench_mlp_api(x_cpu, layers, acts, enc, steps, warmup, rotate=ROTATE):
    """The same chain through the drop-in API, `m(rdv.wrap(x))`, with
    set_synchronous(False) so that calls queue as C ABI launches do: each call
    reads the layers' fp32 parameters afresh (rdv_mlp_forward_unpacked)."""
    import rdv_project_amd as rdv
    m, _, _, xs, _ = _mlp_setup(x_cpu, layers, acts, enc, rotate)
    xw = [rdv.wrap(t) for t in xs]
    prev = rdv.set_synchronous(False)
    try:
        def launch(i):
            m(xw[i % rotate])

        wall, ev = _time_launches(launch, steps, warmup)
    finally:
        rdv.set_synchronous(prev)
    return wall, ev


def bench_winograd(steps, warmup):
    """C3 through the C ABI: NCHW fp16 in / out, ReLU, rotating x / y sets."""
    import torch
    import rdv_project_amd as rdv
    from rdv_project_amd import _conv, _lib
    from rdv_project_amd import workloads as WL
    lib = _lib.load()
    x, w, b = WL.c3()
    conv = rdv.Winograd3x3Conv2d(w.cuda(), b.cuda())
    xd = x.cuda()
    xs = [xd] + [xd.clone() for _ in range(C3_ROTATE - 1)]
    ys = [torch.empty(1, 64, 256, 256, dtype=torch.float16, device="cuda") for _ in range(C3_ROTATE)]
    d = _conv.conv_desc(1, 256, 256, 64, 64, _lib.LAYOUT_CHW, _lib.DTYPE_F16, _lib.LAYOUT_CHW, _lib.DTYPE_F16, True)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    dptr = C.byref(d)
    up = C.c_void_p(conv.U.data_ptr())
    bp = C.c_void_p(conv.bias.data_ptr())
    xp = [C.c_void_p(t.data_ptr()) for t in xs]
    yp = [C.c_void_p(t.data_ptr()) for t in ys]
    fwd = lib.rdv_winograd3x3_forward

    def launch(i):
        k = i % C3_ROTATE
        rc = fwd(dptr, xp[k], up, bp, yp[k], stream)
        if rc != 0:
            _lib.check(rc, "winograd forward")

    wall, ev = _time_launches(launch, steps, warmup)
    return {
        "us_per_call": round(wall * 1e3, 3),
        "kernel_us": round(ev * 1e3, 3),
        "TFLOP_s_direct_equiv": round(C3_DIRECT_FLOP / (ev * 1e-3) / 1e12, 2),
        "TFLOP_s_winograd_mfma": round(C3_WINO_FLOP / (ev * 1e-3) / 1e12, 2),
        "hbm_GB_s": round(C3_BYTES / (ev * 1e-3) / 1e9, 1),
        "hbm_frac": round(C3_BYTES / (ev * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "workload": "C3 Winograd F(2x2,3x3): NCHW fp16 1x64x256x256 U[0,1] (seed 3), 64 -> 64, "
                    "w ~ N(0, sqrt(2/576)) fp16 (seed 4), zero bias, ReLU, fp16 out",
        "kernel": "winograd3x3_pipe_kernel<2>",
    }


def bench_render(steps, warmup):
    """C4: the fused MLP-in-the-loop renderer (one frame per step) and the
    HBM-streaming compositing kernel on C4-sized samples."""
    import torch
    import rdv_project_amd as rdv
    from rdv_project_amd import _chain, _lib, _render
    from rdv_project_amd import workloads as WL
    lib = _lib.load()
    m = None
    for i, (w, b) in enumerate(WL.c4_mlp()):
        lin = rdv.linear(w.cuda(), b.cuda(), f16=True)
        m = lin if m is None else m >> lin
        if i < 3:
            m = m >> rdv.relu
    p = _chain.plan_chain(m, 3)
    packed = _chain.packed_params(m, p)
    cam = rdv.Cameras(WL.C4_WIDTH, WL.C4_HEIGHT, WL.c4_pose().cuda())
    d = _render.camera_desc(cam)
    poses = cam.poses.as_tensor("torch")
    img = torch.empty(1, WL.C4_HEIGHT, WL.C4_WIDTH, 3, device="cuda")
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    dp, pp, pk, ip = C.byref(d), C.c_void_p(poses.data_ptr()), C.c_void_p(packed.data_ptr()), C.c_void_p(img.data_ptr())
    desc = C.byref(p.desc)

    def launch(i):
        rc = lib.rdv_render_emission_absorption(dp, pp, desc, pk, WL.C4_SAMPLES, ip, stream)
        if rc != 0:
            _lib.check(rc, "render")

    wall, ev = _time_launches(launch, steps, warmup)
    # samples actually evaluated: 128 per ray that meets the box
    r = cam().as_tensor("torch").reshape(-1, 6)
    inv = 1.0 / r[:, 3:]
    xc, sa = -r[:, :3] * inv, inv.abs()
    tmin = (xc - sa).max(dim=1).values
    tmax = (xc + sa).min(dim=1).values
    hits = int((~((tmax <= 0) | (tmin > tmax))).sum())
    samples = hits * WL.C4_SAMPLES
    tflops = C4_FLOP_PER_SAMPLE * samples / (ev * 1e-3) / 1e12
    out = {
        "ms_per_frame": round(wall, 4),
        "kernel_ms": round(ev, 4),
        "Msamples_per_s": round(samples / (ev * 1e-3) / 1e6, 1),
        "TFLOP_s": round(tflops, 1),
        "mfma_peak_pct": round(100 * tflops / PEAK_FP16_TFLOPS, 2),
        "hit_rays": hits,
        "workload": "C4 emission-absorption render: 512x512 pinhole rays (origin (0,0,-3.5), target 0, fov pi/4) "
                    "through [-1,1]^3, 128 samples per ray, MLP 3->64->64->64->4 (Kaiming-uniform fp16, seed 2), "
                    "softplus density + sigmoid RGB, front-to-back fp32 compositing, one fused kernel",
        "kernel": "render_ea_kernel",
    }
    # compositing kernel alone over C4-sized samples (262,144 rays x 128)
    nr = WL.C4_WIDTH * WL.C4_HEIGHT
    g = torch.Generator(device="cpu").manual_seed(9)
    sets = [torch.rand(nr, WL.C4_SAMPLES, 4, generator=g).cuda() for _ in range(2)]
    dts = (torch.rand(nr, generator=g) * 0.02).cuda()
    cout = torch.empty(nr, 3, device="cuda")
    sp = [C.c_void_p(t.data_ptr()) for t in sets]
    dtp, cop = C.c_void_p(dts.data_ptr()), C.c_void_p(cout.data_ptr())

    def launch_c(i):
        rc = lib.rdv_composite(sp[i % 2], dtp, C.c_int64(nr), WL.C4_SAMPLES, cop, stream)
        if rc != 0:
            _lib.check(rc, "composite")

    _, cev = _time_launches(launch_c, max(steps, 20), warmup)
    gbs = C4_COMPOSITE_BYTES_PER_RAY * nr / (cev * 1e-3) / 1e9
    out["composite"] = {"kernel_us": round(cev * 1e3, 2), "hbm_GB_s": round(gbs, 1),
                        "hbm_frac": round(gbs / PEAK_HBM_GBS, 4), "bytes_per_ray": C4_COMPOSITE_BYTES_PER_RAY,
                        "rays": nr, "kernel": "composite_kernel<2>"}
    return out


def bench_train(steps, warmup):
    """C5: one training step (forward, MSE, backward, fp32 dW) over 4,194,304 points."""
    import torch
    import rdv_project_amd as rdv
    from rdv_project_amd import workloads as WL
    x, t, layers = WL.c5()
    m = None
    for i, (w, b) in enumerate(layers):
        lin = rdv.linear(w.cuda(), b.cuda(), f16=True)
        m = lin if m is None else m >> lin
        if i + 1 < len(layers):
            m = m >> rdv.relu
    xd, td = x.cuda(), t.cuda()
    loss, grads = rdv.mse_backward(m, xd, td)

    def launch(i):
        rdv.mse_backward(m, xd, td, grads)

    wall, ev = _time_launches(launch, steps, warmup)
    n = x.shape[0]
    tflops = C5_FLOP_PER_POINT * n / (ev * 1e-3) / 1e12
    return {
        "ms_per_step": round(wall, 3),
        "kernel_ms": round(ev, 3),
        "TFLOP_s": round(tflops, 1),
        "mfma_peak_pct": round(100 * tflops / PEAK_FP16_TFLOPS, 2),
        "loss": round(float(loss.item()), 5),
        "workload": "C5 MLP training step: 4,194,304 points x ~ N(0,1) fp16 (seed 5), 32 -> 128 x 8 -> 16, ReLU, "
                    "MSE against N(0,1) targets (seed 6), Kaiming-uniform fp16 weights (seed 7); forward, loss, "
                    "backward with fp32 dW / db reduced over all points",
        "kernels": "train_fwd_pair_kernel x2 (layers 0-4, 5-8) + train_pair2_kernel x4 (layer pairs 8-7 .. 2-1) + "
                   "train_bwd0_kernel (layer 0) + one reduction",
    }


def bench_tensor_ops(steps, warmup):
    """TensorOperation path at the C5 layer shape: LinearTensorOpSmall over
    4,194,304 x 128 -> 128 fp32 rows (x and y each 2 GiB, far beyond the MALL)
    and ReLUTensorOp over the same 4,194,304 x 128 buffer."""
    import torch
    import rdv_project_amd as rdv
    n, inf, outf = 4_194_304, 128, 128
    g = torch.Generator(device="cuda").manual_seed(12)
    x = torch.randn(n, inf, device="cuda", generator=g)
    W = torch.randn(outf, inf, device="cuda", generator=g) / inf ** 0.5
    b = torch.randn(outf, device="cuda", generator=g)
    op = rdv.LinearTensorOpSmall(x, W, b)
    wall, ev = _time_launches(lambda i: op.evaluate(), steps, warmup)
    nbytes = n * (inf + outf) * 4
    relu = rdv.ReLUTensorOp(x)
    rwall, rev = _time_launches(lambda i: relu.evaluate(), steps, warmup)
    rbytes = n * inf * 8
    return {
        "LinearTensorOpSmall": {
            "workload": "4,194,304 x 128 -> 128, fp32 x / y, fp16 operands, fp32 accumulate (seed 12)",
            "ms_per_call": round(wall, 4),
            "kernel_ms": round(ev, 4),
            "GB_s": round(nbytes / (ev * 1e-3) / 1e9, 1),
            "hbm_peak_pct": round(100 * nbytes / (ev * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
            "TFLOP_s": round(2.0 * n * inf * outf / (ev * 1e-3) / 1e12, 1),
            "bytes_per_call": nbytes,
            "kernel": "linear_op_kernel<true, 2, 4>",
        },
        "ReLUTensorOp": {
            "workload": "4,194,304 x 128 fp32",
            "kernel_ms": round(rev, 4),
            "GB_s": round(rbytes / (rev * 1e-3) / 1e9, 1),
            "hbm_peak_pct": round(100 * rbytes / (rev * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
            "kernel": "relu_op_kernel",
        },
    }


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def _median_time(fn, warm: int = 3, runs: int = 5) -> float:
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(runs):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return statistics.median(ts)


def bench_conv_and_data_ops(steps, warmup):
    """The direct-convolution kernel (rdv_conv2d, fp16 operands) at the C3
    shape in the tensor-op layout (channels-last fp32 x and y, 256 x 256,
    64 -> 64, 3x3), and the data-movement ops at C3-sized images."""
    import torch
    from rdv_project_amd import _lib, _tensor_ops
    from rdv_project_amd import workloads as WL
    H = W = 256
    C = K = 64
    g = WL.gen(15)
    x = (torch.rand(H * W, C, generator=g) * 2 - 1).cuda()
    w = (torch.randn(3, 3, C, K, generator=g) * (2.0 / (9 * C)) ** 0.5).cuda()
    b = torch.zeros(K).cuda()
    ys = [torch.empty(H * W, K, device="cuda") for _ in range(4)]
    xs = [x] + [x.clone() for _ in range(3)]
    d = _tensor_ops.conv2d_desc(H, W, C, K, 3, 3, _lib.PREC_F16, _lib.WLAYOUT_RSCK)
    wall, ev = _time_launches(lambda i: _tensor_ops.conv2d(d, xs[i % 4], w, b, ys[i % 4], "conv"), steps, warmup)
    flop = 2 * H * W * C * K * 9
    nbytes = H * W * (C + K) * 4
    out = {"direct_conv": {
        "workload": "implicit-GEMM direct conv, fp16 operands: channels-last fp32 x [256*256, 64] (seed 15), "
                    "3x3 64 -> 64, 'same' padding, fp32 y (Conv2DTensorOp{Fast,Simple,Simple3x3,Window3x3})",
        "kernel": "conv_tile_kernel<4>",
        "us_per_call": round(ev * 1e3, 2),
        "TFLOP_s": round(flop / (ev * 1e-3) / 1e12, 1),
        "mfma_peak_pct": round(100 * flop / (ev * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 2),
        "hbm_GB_s": round(nbytes / (ev * 1e-3) / 1e9, 1),
        "hbm_peak_pct": round(100 * nbytes / (ev * 1e-3) / 1e9 / PEAK_HBM_GBS, 2),
        "bytes_per_call": nbytes,
    }}
    big = [(torch.rand(H * W, C, generator=g)).cuda() for _ in range(4)]
    small = [torch.empty(H * W // 4, C, device="cuda") for _ in range(4)]
    up_out = [torch.empty(H * W, C, device="cuda") for _ in range(4)]
    cat_out = [torch.empty(H * W, 2 * C, device="cuda") for _ in range(2)]
    _, ev_d = _time_launches(lambda i: _tensor_ops.downsample2x(big[i % 4], H, W, small[i % 4]), steps, warmup)
    _, ev_u = _time_launches(lambda i: _tensor_ops.upsample2x(small[i % 4], H // 2, W // 2, up_out[i % 4]),
                             steps, warmup)
    _, ev_c = _time_launches(lambda i: _tensor_ops.concat(big[i % 4], big[(i + 1) % 4], cat_out[i % 2]), steps, warmup)
    img = H * W * C * 4
    for name, evx, nb, kern in (("downsample2x", ev_d, img + img // 4, "downsample2x_kernel<uint32_t>"),
                                ("upsample2x", ev_u, img // 4 + img, "upsample2x_kernel<uint32_t>"),
                                ("concat", ev_c, 4 * img, "concat_kernel<uint32_t>")):
        gbs = nb / (evx * 1e-3) / 1e9
        out[name] = {"us_per_call": round(evx * 1e3, 2), "hbm_GB_s": round(gbs, 1),
                     "hbm_peak_pct": round(100 * gbs / PEAK_HBM_GBS, 2), "bytes_per_call": nb, "kernel": kern,
                     "workload": "256 x 256 x 64 fp32 channels-last image (seed 15)"}
    return out


def cpu_baseline():
    """The torch-CPU restatement (oracle/torch_cpu.py) on the host cores: C1 in
    full, bounded samples of C2 (2^18 points), C3 (the whole 256x256 image), C4
    (4,096 rays x 128 samples) and C5 (2^16 points, forward + backward); each a
    median of 5 after 3 warm-ups, data generation excluded."""
    import torch
    from oracle import torch_cpu as TC
    from rdv_project_amd import workloads as WL
    cores = len(os.sched_getaffinity(0))
    prev_threads = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        with torch.no_grad():
            n2 = 1 << 18
            x2, l2 = WL.c2(n2)
            p2 = TC.pack_layers(l2)
            t2 = _median_time(lambda: TC.mlp_forward(x2, p2, ["relu"] * 3 + ["none"], (WL.C2_OCTAVES, WL.C2_PAD)))
            x1, l1 = WL.c1()
            p1 = TC.pack_layers(l1)
            t1 = _median_time(lambda: TC.mlp_forward(x1, p1, ["relu"] * 4 + ["none"]))
            x3, w3, _ = WL.c3()
            x3f, w3f = x3.float(), w3.float()
            t3 = _median_time(lambda: TC.conv3x3(x3f, w3f, relu=True), warm=1, runs=3)
            p4 = TC.pack_layers(WL.c4_mlp())
            g = torch.Generator().manual_seed(0)
            rays = torch.cat([torch.tensor([[0.0, 0.0, -3.5]]).expand(4096, 3),
                              torch.nn.functional.normalize(torch.randn(4096, 3, generator=g) * 0.15 +
                                                            torch.tensor([0.0, 0.0, 1.0]), dim=1)], dim=1)
            t4 = _median_time(lambda: TC.render_ea(rays, p4, WL.C4_SAMPLES), warm=1, runs=3)
        n5 = 1 << 16
        x5, tg5, l5 = WL.c5(n5)
        x5f = x5.float()
        params = [(w.clone().requires_grad_(True), b.clone().requires_grad_(True)) for w, b in l5]
        t5 = _median_time(lambda: TC.train_step(x5f, tg5, params), warm=1, runs=3)
    finally:
        torch.set_num_threads(prev_threads)
    return {
        "value": round(n2 / t2 / 1e6, 3),
        "unit": "Mpoints/s",
        "cores": cores,
        "kind": "port",
        "sample": f"C2 forward on {n2} of the 2^20 points: torch-CPU fp32 GEMMs on fp16-rounded operands "
                  f"(oracle/torch_cpu.py), torch threads = {cores}, median of 5 after 3 warm-ups",
        "cpu_model": _cpu_model(),
        "per_config": {
            "C1_full_Mpoints_per_s": round(x1.shape[0] / t1 / 1e6, 3),
            "C2_sample_Mpoints_per_s": round(n2 / t2 / 1e6, 3),
            "C3_full_TFLOP_s_direct_equiv": round(C3_DIRECT_FLOP / t3 / 1e12, 4),
            "C4_sample_Msamples_per_s": round(4096 * WL.C4_SAMPLES / t4 / 1e6, 3),
            "C5_sample_Mpoints_per_s": round(n5 / t5 / 1e6, 4),
            "C5_sample_TFLOP_s": round(C5_FLOP_PER_POINT * n5 / t5 / 1e12, 4),
        },
    }


def bench_generic_mlp(steps, warmup):
    """The runtime-shaped matrix-core MLP (a chain without a compile-time
    instance): 2^20 points U[-1,1]^64 (seed 13), 64 -> 128 -> 128 -> 128 -> 16,
    ReLU, Kaiming-uniform fp16 weights (seed 14)."""
    import torch
    from rdv_project_amd import workloads as WL
    n = 1 << 20
    x = torch.rand(n, GEN_DIMS[0], generator=WL.gen(13)) * 2.0 - 1.0
    layers = WL.kaiming_uniform_f16([(GEN_DIMS[i + 1], GEN_DIMS[i]) for i in range(len(GEN_DIMS) - 1)], seed=14)
    acts = ["relu"] * (len(layers) - 1) + ["none"]
    wall, ev, name = bench_mlp(x, layers, acts, None, steps, warmup, rotate=4)
    tflops = GEN_FLOP_PER_POINT * n / (ev * 1e-3) / 1e12
    return {
        "workload": "runtime-shaped LinearFast chain: 2^20 points U[-1,1]^64 (seed 13), 64 -> 128 -> 128 -> 128 -> 16, "
                    "ReLU, Kaiming-uniform fp16 weights (seed 14), fp32 accumulate, one kernel",
        "kernel": name,
        "us_per_call": round(ev * 1e3, 2),
        "wall_us_per_call": round(wall * 1e3, 2),
        "Mpoints_per_s": round(n / (ev * 1e-3) / 1e6, 1),
        "TFLOP_s": round(tflops, 1),
        "mfma_peak_pct": round(100 * tflops / PEAK_FP16_TFLOPS, 2),
        "flop_per_point": GEN_FLOP_PER_POINT,
    }


def bench_f32_chain(steps, warmup):
    """The exact-fp32 Linear chain (Linear layers, every product and sum in fp32 in the reference's order):
    C1's network and points, 3 -> 64 -> 64 -> 64 -> 64 -> 4, ReLU, 65,536 points."""
    from rdv_project_amd import workloads as WL
    x, layers = WL.c1()
    n = x.shape[0]
    acts = ["relu"] * 4 + ["none"]
    wall, ev, name = bench_mlp(x, layers, acts, None, steps, warmup, rotate=4, f16=False)
    flop = C1_FLOP_PER_POINT * n
    return {
        "workload": "exact-fp32 Linear chain: C1's 65,536 points U[-1,1]^3 (seed 0), 3 -> 64 -> 64 -> 64 -> 64 -> 4, "
                    "ReLU, Kaiming-uniform weights (seed 1), fp32 products and sums in the reference's order",
        "kernel": name,
        "us_per_call": round(ev * 1e3, 2),
        "wall_us_per_call": round(wall * 1e3, 2),
        "Mpoints_per_s": round(n / (ev * 1e-3) / 1e6, 1),
        "TFLOP_s": round(flop / (ev * 1e-3) / 1e12, 2),
        "fp32_vector_peak_pct": round(100 * flop / (ev * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 2),
    }


def bench_volumes(steps, warmup):
    """Ratio-tracking transmittance (RatiotrackingTransmittance with a VoxelMajorantField) over the C4 camera's
    512 x 512 rays: extinction = a 3 -> 64 -> 64 -> 64 -> 1 softplus LinearFast chain (Kaiming-uniform fp16,
    seed 11), density_scale 4, majorant = MajorantGrid(64^3 lattice of the extinction x 1.3, [8, 8, 8])."""
    import torch
    import rdv_project_amd as rdv
    from rdv_project_amd import _chain, _lib, _render
    from rdv_project_amd import workloads as WL
    from rdv_project_amd.types import RandomLibrary
    lib = _lib.load()
    layers = WL.kaiming_uniform_f16([(64, 3), (64, 64), (64, 64), (1, 64)], seed=11)
    ext = None
    for i, (w, b) in enumerate(layers):
        lin = rdv.linear(w.cuda(), b.cuda(), f16=True)
        ext = lin if ext is None else ext >> lin
        ext = ext >> (rdv.relu if i + 1 < len(layers) else rdv.softplus)
    c = (torch.arange(64, dtype=torch.float32) + 0.5) / 64 * 2 - 1
    zz, yy, xx = torch.meshgrid(c, c, c, indexing="ij")
    lattice = torch.stack([xx, yy, zz], -1).reshape(-1, 3).cuda()
    dens = ext(rdv.wrap(lattice)).as_tensor("torch").reshape(64, 64, 64, 1) * 1.3 + 1e-3
    mg = rdv.MajorantGrid(rdv.TensorGrid(dens.clone()), [8, 8, 8])
    rt = rdv.RatiotrackingTransmittance(ext, mg, density_scale=4.0)
    majv = mg().as_tensor("torch").contiguous().clone()
    p = _chain.plan_chain(ext, 3)
    packed = _chain.packed_params(ext, p)
    rays = rdv.Cameras(WL.C4_WIDTH, WL.C4_HEIGHT, WL.c4_pose().cuda())().as_tensor("torch").reshape(-1, 6).clone()
    n = rays.shape[0]
    out = torch.empty(n, device="cuda")
    RandomLibrary.seed(0)
    d = _render._ratio_desc(rt, RandomLibrary.next_seeds(), 0, 8, 8, 8)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (C.byref(p.desc), C.c_void_p(packed.data_ptr()), C.byref(d), C.c_void_p(majv.data_ptr()),
            C.c_void_p(rays.data_ptr()), C.c_int64(n), C.c_void_p(out.data_ptr()), stream)

    def launch(i):
        d.seeds[0] = 128 + i  # a fresh generator per call, as each dispatch draws new seeds
        rc = lib.rdv_ratiotracking_transmittance(*args)
        if rc != 0:
            _lib.check(rc, "ratio tracking")

    wall, ev = _time_launches(launch, steps, warmup)
    T = out.double()
    # majorant grid alone (64^3 -> 8^3, linear, unaligned): 1 MiB read per call
    fine = dens.contiguous()
    mout = torch.empty(8, 8, 8, 1, device="cuda")
    gd = _lib.MajorantGridDesc()
    gd.rank, gd.channels, gd.aligned, gd.linear = 3, 1, 0, 1
    for i in range(3):
        gd.fine_shape[i], gd.shape[i] = 64, 8

    def launch_mg(i):
        rc = lib.rdv_majorant_grid(C.byref(gd), C.c_void_p(fine.data_ptr()), C.c_void_p(mout.data_ptr()), stream)
        if rc != 0:
            _lib.check(rc, "majorant grid")

    _, mev = _time_launches(launch_mg, max(steps, 20), warmup, prewarm_s=0.05)

    # RaymarchingTransmittance over the same rays and extinction (fixed steps of 0.002, cut at tau > 16)
    tarr = (C.c_float * 12)(1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0)
    tout = torch.empty(n, device="cuda")

    def launch_rm(i):
        rc = lib.rdv_raymarch_transmittance(C.byref(p.desc), C.c_void_p(packed.data_ptr()),
                                            C.c_void_p(rays.data_ptr()), C.c_int64(n), tarr, C.c_float(0.002),
                                            C.c_float(4.0), C.c_void_p(tout.data_ptr()), stream)
        if rc != 0:
            _lib.check(rc, "raymarching transmittance")

    _, rev = _time_launches(launch_rm, max(steps, 20), warmup)
    return {
        "workload": "ratio tracking over 512x512 C4 camera rays, extinction 3->64->64->64->1 softplus (fp16 MFMA, "
                    "seed 11), density_scale 4, 8^3 voxel majorant from a 64^3 MajorantGrid",
        "raymarch": {"workload": "RaymarchingTransmittance over the same rays and extinction, step 0.002, "
                                 "density_scale 4 (fixed steps, cut at tau > 16)",
                     "kernel": "raymarch_transmittance_kernel",
                     "ms_per_call": round(rev, 4), "Mrays_per_s": round(n / (rev * 1e-3) / 1e6, 1),
                     "mean_T": round(float(tout.double().mean()), 4)},
        "kernel": "ratiotracking_generic_kernel",
        "ms_per_call": round(ev, 4),
        "Mrays_per_s": round(n / (ev * 1e-3) / 1e6, 1),
        "mean_T": round(float(T.mean()), 4),
        "majorant_grid_us": round(mev * 1e3, 2),
        "bound": "per-ray free-flight loop; one chain evaluation per collision for the 32 rays of a wave",
    }


def main() -> int:
    global PREWARM_S
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU baseline (profiling runs)")
    ap.add_argument("--no-extras", action="store_true", help="only the headline configuration")
    ap.add_argument("--prewarm", type=float, default=PREWARM_S,
                    help="seconds of untimed launches before each configuration's warm-up (0 for counter runs)")
    ap.add_argument("--calib-copy", action="store_true",
                    help="first run 5 plain 64 MiB device copies (known HBM bytes) so that a rocprofv3 --pmc "
                         "FETCH_SIZE / WRITE_SIZE run can scale the counters")
    args = ap.parse_args()
    PREWARM_S = max(0.0, args.prewarm)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: every box of this run has a single MI355X, and the hot path "
              "(independent points / rays / image tiles) needs no collective. Run with --gpus 1.",
              file=sys.stderr)
        return 2

    import torch
    import rdv_project_amd as rdv
    from rdv_project_amd import workloads as WL

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    torch.cuda.set_device(0)
    rdv.set_synchronous(False)

    if args.calib_copy:
        src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---------------------------------------------------------------- C2 headline
    _log("C2 setup")
    x, layers = WL.c2()
    enc = rdv.FrequencyEncoding(3, WL.C2_OCTAVES, pad_to=WL.C2_PAD)
    acts = ["relu"] * 3 + ["none"]
    wall, ev, kname = bench_mlp(x, layers, acts, enc, args.steps, args.warmup)
    n = x.shape[0]
    mpts = n / (ev * 1e-3) / 1e6
    achieved = C2_FLOP_PER_POINT * n / (ev * 1e-3) / 1e12
    _log(f"C2 {kname}: events {ev * 1e3:.2f} us/step, wall {wall * 1e3:.2f} us/step, "
         f"{mpts:.0f} Mpts/s, {achieved:.1f} TFLOP/s")

    extras = {}
    _log("C2 through the API")
    aw, ae = bench_mlp_api(x, layers, acts, enc, args.steps, args.warmup)
    extras["C2_api"] = {
        "call": "m(rdv.wrap(x)) with set_synchronous(False): plan cached on the map, one rdv_mlp_forward_unpacked "
                "launch converting the layers' fp32 parameters in the kernel",
        "us_per_call": round(ae * 1e3, 3),
        "wall_us_per_call": round(aw * 1e3, 3),
        "Mpoints_per_s": round(n / (ae * 1e-3) / 1e6, 1),
        "vs_c_abi_ms_per_step": round(ae / ev, 4),
    }
    _log(f"C2 API {extras['C2_api']}")
    if not args.no_extras:
        _log("C1")
        x1, l1 = WL.c1()
        w1, e1, k1 = bench_mlp(x1, l1, ["relu"] * 4 + ["none"], None, max(args.steps // 2, 10), args.warmup)
        extras["C1_fused_mlp"] = {
            "Mpoints_per_s": round(x1.shape[0] / (e1 * 1e-3) / 1e6, 1),
            "kernel_us": round(e1 * 1e3, 3),
            "wall_us_per_call": round(w1 * 1e3, 3),
            "TFLOP_s": round(C1_FLOP_PER_POINT * x1.shape[0] / (e1 * 1e-3) / 1e12, 2),
            "kernel": k1,
        }
        _log("C3")
        extras["C3_winograd"] = bench_winograd(max(args.steps // 2, 10), args.warmup)
        _log(f"C3 {extras['C3_winograd']}")
        _log("C4")
        extras["C4_render"] = bench_render(max(args.steps // 50, 10), 3)
        _log(f"C4 {extras['C4_render']}")
        _log("C5")
        rdv.set_synchronous(False)
        extras["C5_train"] = bench_train(5, 2)
        _log(f"C5 {extras['C5_train']}")
        _log("tensor ops")
        extras["tensor_ops"] = bench_tensor_ops(20, 3)
        _log(f"tensor ops {extras['tensor_ops']}")
        _log("conv and data ops")
        extras.update(bench_conv_and_data_ops(max(args.steps // 5, 10), args.warmup))
        _log(f"conv {extras['direct_conv']}")
        _log("generic MLP")
        extras["generic_mlp"] = bench_generic_mlp(max(args.steps // 5, 10), args.warmup)
        _log(f"generic MLP {extras['generic_mlp']}")
        extras["f32_chain"] = bench_f32_chain(max(args.steps // 20, 10), 3)
        _log(f"fp32 chain {extras['f32_chain']}")
        _log("ratio tracking")
        extras["ratiotracking"] = bench_volumes(max(args.steps // 20, 10), 3)
        _log(f"ratio tracking {extras['ratiotracking']}")
        extras["volume_profile"] = bench_volume_profile(3, 1)
        _log(f"volume profile {extras['volume_profile']}")

    cpu = None
    if not args.no_cpu_baseline:
        _log("CPU baseline (torch-CPU restatement, bounded samples)")
        cpu = cpu_baseline()
        _log(f"CPU baseline {cpu}")

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "mlp_fused_c2_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC,
        "value": round(mpts, 1),
        "unit": "Mpoints/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ev, 6),
        "wall_ms_per_step": round(wall, 6),
        "clock": "hip_events on the launch stream around the K timed steps (value, ms_per_step, roofline)",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": "C2 encoded coordinate MLP: 2^20 points U[-1,1]^3 (seed 0), FREQ 6 octaves "
                        "(39 features, zero padded to 48) -> 64 -> 64 -> 64 -> 4, ReLU, Kaiming-uniform fp16 "
                        "weights (seed 1), fp32 accumulate, one fused kernel",
            "points": n,
            "kernel": kname,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
            "traffic": traffic,
            "traffic_source": "profiles/mlp_fused_c2_traffic.json: two rocprofv3 --pmc runs of this command "
                              "(FETCH_SIZE, WRITE_SIZE) scaled by a copy kernel of known size",
        },
        "mfma_peak_pct": round(100.0 * achieved / PEAK_FP16_TFLOPS, 2),
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
