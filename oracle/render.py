"""Oracle for cameras, MLP-in-the-loop volume rendering and compositing —
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference semantics restated (paths relative to /root/reference/src/rdv):
  * Cameras (domain/rendering.py:10-42, shaders/rendering/cameras.h:1-20): for
    camera c and pixel (x, y) of a W x H image, p = ((x, y) + 0.5) / (W, H) * 2 - 1,
    s = (p.x * aspect, p.y, 1 / tan(fov / 2)), z = normalize(target - origin),
    x_axis = normalize(cross(up, z)), y_axis = cross(z, x_axis),
    w = normalize(s.x x_axis + s.y y_axis + s.z z); the ray is (origin, w).
    Defaults: aspect = W / H, fov = pi / 4 (rendering.py:31-34).
  * ray_box_intersection (shaders/libraries/math_library.h:48-57) against
    [-1, 1]^3: inv = 1 / w, xc = -x inv, s = |inv|, tMin = max(xc - s),
    tMax = min(xc + s).
  * RaymarchingTransmittance (domain/volumes.py:124-141,
    shaders/volumes/raymarching_transmittance.h:1-22,
    raymarching_transmittance_trait.h:1-14): object space x = L (x - O), w = L w
    with L = inverse of the transform's linear part; a miss (tMax <= 0 or
    tMin > tMax) gives 1; else x += w max(0, tMin), d = tMax - max(0, tMin) and
        for k = 0; d > 0 and k < 4096; k++:
            tau += extinction(x) * density_scale * step;  if tau > 16: return 0
            d -= step;  x += step * w
        return exp(-tau)
    every operation rounded to fp32 (restated here in numpy float32, the
    product and the sum rounded separately).
  * Emission-absorption (build-defined, no reference counterpart): S samples
    t_i = t0 + (i + 1/2) dt, dt = (t1 - t0) / S on [t0, t1] = [max(0, tMin), tMax],
    (sigma, c) = (softplus(o_0), sigmoid(o_1..3)) of the field at o + t_i w,
    alpha_i = 1 - exp(-sigma_i dt), T_i = prod_{j<i} (1 - alpha_j),
    C = sum_i T_i alpha_i c_i; 0 for rays that miss.  Compositing in float64.

The field MLPs are evaluated with oracle.mlp.chain on every sample in fp16
(LinearFast) arithmetic: the GPU evaluates samples in full 32-sample matrix-core
blocks, so the partial-workgroup fp32 rule of Map.__call__ does not apply.
"""
from __future__ import annotations

import math

import numpy as np

from . import mlp as M


def _normalize(v):
    return v / np.sqrt(np.sum(v * v, axis=-1, keepdims=True))


def camera_rays(width: int, height: int, poses, aspect: float | None = None, fov: float | None = None,
                jitter: np.ndarray | None = None) -> np.ndarray:
    """[n, H, W, 6] rays (float64) of cameras.h for poses [n, 9].  jitter:
    [n, H, W, 2] sub-pixel positions (x, y) in [0, 1) replacing the centre
    (cameras.h:7: two random() draws per cell when pixel_jitter is set)."""
    poses = np.asarray(poses, np.float64).reshape(-1, 9)
    n = poses.shape[0]
    aspect = width / height if aspect is None else aspect
    fov = math.pi / 4 if fov is None else fov
    o, t, up = poses[:, 0:3], poses[:, 3:6], poses[:, 6:9]
    if jitter is None:
        jitter = np.full((n, height, width, 2), 0.5)
    jitter = np.asarray(jitter, np.float64).reshape(n, height, width, 2)
    xs = (np.arange(width)[None, None, :] + jitter[..., 0]) / width * 2 - 1
    ys = (np.arange(height)[None, :, None] + jitter[..., 1]) / height * 2 - 1
    sx = xs * aspect
    sy = ys
    sz = 1.0 / math.tan(fov * 0.5)
    z = _normalize(t - o)
    xa = _normalize(np.cross(up, z))
    ya = np.cross(z, xa)
    w = (xa[:, None, None, :] * sx[..., None] + ya[:, None, None, :] * sy[..., None] +
         z[:, None, None, :] * sz)
    w = _normalize(w)
    out = np.empty((n, height, width, 6))
    out[..., 0:3] = o[:, None, None, :]
    out[..., 3:6] = w
    return out


def ray_box(x, w):
    """(tMin, tMax) of math_library.h's slab test against [-1, 1]^3.  A ray
    parallel to a slab through its centre plane gives 0 * inf = NaN for that
    axis; max / min ignore it (IEEE maxNum / minNum, the GPU's fmax / fmin), which
    leaves that slab unconstraining, as the geometry says."""
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = 1.0 / w
        xc = -x * inv
        s = np.abs(inv)
        return np.fmax.reduce(xc - s, axis=-1), np.fmin.reduce(xc + s, axis=-1)


def ray_box32(x, w):
    """ray_box with every operation rounded to float32 (the shader's arithmetic)."""
    x = np.asarray(x, np.float32)
    w = np.asarray(w, np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = (np.float32(1) / w).astype(np.float32)
        xc = (-x * inv).astype(np.float32)
    s = np.abs(inv)
    with np.errstate(invalid="ignore"):
        c0 = (xc - s).astype(np.float32)
        c1 = (xc + s).astype(np.float32)
    return np.fmax.reduce(c0, axis=-1), np.fmin.reduce(c1, axis=-1)


def field_eval(p: np.ndarray, layers, acts, precs=None) -> np.ndarray:
    """The field chain on points p [..., 3]: every row with each layer's own
    arithmetic (precs: 'f16' LinearFast, 'f32' Linear; all 'f16' by default)."""
    shp = p.shape[:-1]
    y = M.chain(p.reshape(-1, 3), layers, acts, precs or ["f16"] * len(layers))
    return y.reshape(*shp, -1)


def render_ea(rays: np.ndarray, layers, samples: int, chunk_rays: int = 512) -> np.ndarray:
    """Emission-absorption colour [N, 3] of rays [N, 6] through the field
    (layers: 3 -> ... -> 4, ReLU hidden, raw head)."""
    rays = np.asarray(rays, np.float64).reshape(-1, 6)
    acts = ["relu"] * (len(layers) - 1) + ["none"]
    out = np.zeros((rays.shape[0], 3))
    tmin, tmax = ray_box(rays[:, 0:3], rays[:, 3:6])
    hit = ~((tmax <= 0) | (tmin > tmax))
    idx = np.nonzero(hit)[0]
    for s0 in range(0, idx.size, chunk_rays):
        ii = idx[s0:s0 + chunk_rays]
        t0 = np.maximum(tmin[ii], 0.0)
        dt = (tmax[ii] - t0) / samples
        t = t0[:, None] + (np.arange(samples)[None, :] + 0.5) * dt[:, None]
        p = rays[ii, None, 0:3] + t[..., None] * rays[ii, None, 3:6]
        o = field_eval(p.astype(np.float32), layers, acts).astype(np.float64)
        sigma = np.logaddexp(0.0, o[..., 0])
        c = 1.0 / (1.0 + np.exp(-o[..., 1:4]))
        out[ii] = composite(np.concatenate([sigma[..., None], c], axis=-1), dt)
    return out


def composite(sigma_rgb: np.ndarray, dt: np.ndarray) -> np.ndarray:
    """C = sum_i T_i alpha_i c_i with alpha_i = 1 - exp(-sigma_i dt) and
    T_i = prod_{j<i} (1 - alpha_j), in float64.  sigma_rgb [N, S, 4], dt [N]."""
    s = np.asarray(sigma_rgb, np.float64)
    dt = np.asarray(dt, np.float64)
    a = s[..., 0] * dt[:, None]
    one_minus = np.exp(-a)
    alpha = 1.0 - one_minus
    T = np.cumprod(np.concatenate([np.ones((s.shape[0], 1)), one_minus[:, :-1]], axis=1), axis=1)
    return np.sum((T * alpha)[..., None] * s[..., 1:4], axis=1)


def raymarch_transmittance(rays: np.ndarray, layers, head: str = "softplus", transform=None, step: float = 0.002,
                           density_scale: float = 1.0, precs=None) -> np.ndarray:
    """transmittance_rm per ray [N, 6], the reference's sequential loop in
    float32 (vectorised over rays).  head: activation of the extinction's last
    layer; precs: each layer's arithmetic ('f16' / 'f32', all 'f16' by default)."""
    f = np.float32
    rays = np.asarray(rays, np.float32).reshape(-1, 6)
    Mt = np.eye(4, 3, dtype=np.float64) if transform is None else np.asarray(transform, np.float64).reshape(4, 3)
    lin = Mt[0:3].T                       # columns 0..2 are the linear part
    L = np.linalg.inv(lin).astype(np.float32)
    O = Mt[3].astype(np.float32)
    x = ((rays[:, 0:3] - O) @ L.T).astype(np.float32)
    w = (rays[:, 3:6] @ L.T).astype(np.float32)
    tmin, tmax = ray_box32(x, w)
    out = np.ones(rays.shape[0], np.float64)
    hit = ~((tmax <= 0) | (tmin > tmax))
    tmin = np.maximum(f(0), tmin)
    x = (x + (w * tmin[:, None]).astype(np.float32)).astype(np.float32)
    d = (tmax - tmin).astype(np.float32)
    step = f(step)
    sw = (step * w).astype(np.float32)
    tau = np.zeros(rays.shape[0], np.float32)
    alive = hit.copy()
    dead = np.zeros(rays.shape[0], bool)
    acts = ["relu"] * (len(layers) - 1) + [head]
    for k in range(4096):
        act = alive & (d > 0)
        if not act.any():
            break
        ii = np.nonzero(act)[0]
        sig = field_eval(x[ii], layers, acts, precs)[:, 0].astype(np.float32)
        ce = (sig * f(density_scale)).astype(np.float32)
        tau[ii] = (tau[ii] + (ce * step).astype(np.float32)).astype(np.float32)
        over = tau[ii] > 16
        dead[ii[over]] = True
        alive[ii[over]] = False
        d[ii] = (d[ii] - step).astype(np.float32)
        x[ii] = (x[ii] + sw[ii]).astype(np.float32)
    out[hit] = np.exp(-tau[hit].astype(np.float64))
    out[dead] = 0.0
    return out
