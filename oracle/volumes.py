"""Oracle for voxel majorant fields, majorant grids and ratio-tracking
transmittance — TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Reference semantics restated (paths relative to /root/reference/src/rdv):
  * VoxelMajorantField (domain/volumes.py:191-211,
    shaders/volumes/voxel_majorant_field.h:6-33): for a grid of shape [D, H, W],
    dim = (W, H, D), cell = clamp(int((x * 0.5 + 0.5) * dim), 0, dim - 1)
    (int() truncating), majorant = grid[cell.z, cell.y, cell.x],
    voxel = 2 / dim, bmin = cell * voxel - 1, bmax = bmin + voxel,
    distance = min over axes of max((bmin - x) / w, (bmax - x) / w).
  * MajorantGrid (maths/__init__.py:534-569, shaders/grids/majorant_grid.h):
    per coarse cell i of n along each dimension, t = i / n and (i + 1) / n,
    pos = t (fine - 1) when aligned else t fine - 0.5; linear: [floor(pos_lo),
    floor(pos_hi) + 2), nearest: [floor(pos_lo + 0.5), floor(pos_hi + 0.5) + 1),
    clamped into [0, fine) and kept non-empty; the cell's value is the
    channel-wise max over the product of these ranges.
  * RatiotrackingTransmittance (domain/volumes.py:144-190,
    shaders/volumes/ratiotracking_transmittance.h:1-22,
    ratiotracking_transmittance_trait.h:1-31): object space as
    RaymarchingTransmittance (miss: 1), then
        for safety in 0..1023 while d > 0:
            maj = max(majorant, 1e-12); dist = max(distance, 1e-6)
            dt = min(dist, -log(1 - random()) / (maj * density_scale))
            d -= dt; x += dt * w
            if dt >= dist: continue
            if d <= 0: break
            T *= 1 - extinction(x) / maj
            if T < 0.05: (random() >= T -> return 0) else T = 1
        return T
    with ray i drawing from thread i's generator (oracle.random).
All arithmetic in float32, each operation rounded on its own, vectorised over
rays (every live ray runs one loop iteration per pass, so `safety` is the pass
number).
"""
from __future__ import annotations

import numpy as np

from . import random as RNG
from .render import field_eval, ray_box32

F = np.float32


def voxel_majorant(grid: np.ndarray, x: np.ndarray, w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(majorant [n], distance [n]) of rays (x, w) [n, 3] in a grid [D, H, W]."""
    grid = np.asarray(grid, F)
    D, H, W = grid.shape[:3]
    x = np.asarray(x, F)
    w = np.asarray(w, F)
    dim = np.array([W, H, D], F)
    f = ((x * F(0.5) + F(0.5)).astype(F) * dim).astype(F)
    with np.errstate(invalid="ignore"):
        cell = np.clip(np.trunc(np.nan_to_num(f, nan=0.0, posinf=1e9, neginf=-1e9)), 0, dim - 1).astype(np.int64)
    vs = (F(2.0) / dim).astype(F)
    bmin = (cell.astype(F) * vs - F(1.0)).astype(F)
    bmax = (bmin + vs).astype(F)
    with np.errstate(divide="ignore", invalid="ignore"):
        t0 = ((bmin - x).astype(F) / w).astype(F)
        t1 = ((bmax - x).astype(F) / w).astype(F)
    te = np.fmax(t0, t1)
    dist = np.fmin(np.fmin(te[:, 0], te[:, 1]), te[:, 2])
    maj = grid.reshape(D, H, W)[cell[:, 2], cell[:, 1], cell[:, 0]]
    return maj.astype(F), dist.astype(F)


def _range(i: int, n: int, fine: int, aligned: bool, linear: bool) -> tuple[int, int]:
    fsz = F(fine)
    t_lo = F(F(i) / F(n))
    t_hi = F(F(i + 1) / F(n))
    if aligned:
        pos_lo, pos_hi = F(t_lo * F(fsz - F(1))), F(t_hi * F(fsz - F(1)))
    else:
        pos_lo, pos_hi = F(F(t_lo * fsz) - F(0.5)), F(F(t_hi * fsz) - F(0.5))
    if linear:
        lo, hi = int(np.floor(pos_lo)), int(np.floor(pos_hi)) + 2
    else:
        lo, hi = int(np.floor(F(pos_lo + F(0.5)))), int(np.floor(F(pos_hi + F(0.5)))) + 1
    lo = max(lo, 0)
    hi = min(hi, fine)
    if hi <= lo:
        hi = lo + 1
    hi = min(hi, fine)
    if lo >= hi:
        lo = hi - 1
    return lo, hi


def majorant_grid(fine: np.ndarray, shape, aligned: bool = False, linear: bool = True) -> np.ndarray:
    """MajorantGrid values [*shape, C] of fine values [*fine_shape, C]."""
    fine = np.asarray(fine, F)
    rank = len(shape)
    C = fine.shape[-1]
    ranges = [[_range(i, int(shape[d]), int(fine.shape[d]), aligned, linear) for i in range(int(shape[d]))]
              for d in range(rank)]
    out = np.empty((*shape, C), F)
    for idx in np.ndindex(*shape):
        sl = tuple(slice(*ranges[d][idx[d]]) for d in range(rank))
        out[idx] = fine[sl].reshape(-1, C).max(axis=0)
    return out


def object_space(rays: np.ndarray, transform=None):
    """(x, w, d, hit) of rays [n, 6] at their box entry (RaymarchingTransmittance's set-up)."""
    rays = np.asarray(rays, F).reshape(-1, 6)
    Mt = np.eye(4, 3, dtype=np.float64) if transform is None else np.asarray(transform, np.float64).reshape(4, 3)
    L = np.linalg.inv(Mt[0:3].T).astype(F)
    O = Mt[3].astype(F)
    x = ((rays[:, 0:3] - O) @ L.T).astype(F)
    w = (rays[:, 3:6] @ L.T).astype(F)
    tmin, tmax = ray_box32(x, w)
    hit = ~((tmax <= 0) | (tmin > tmax))
    tmin = np.maximum(F(0), tmin)
    x = (x + (w * tmin[:, None]).astype(F)).astype(F)
    d = (tmax - tmin).astype(F)
    return x, w, d, hit


def ratiotracking(rays: np.ndarray, extinction, majorant: np.ndarray, seeds, transform=None,
                  density_scale: float = 1.0, rng_skip: int = 0) -> np.ndarray:
    """Ratio-tracking transmittance [n] (float32) of rays [n, 6].  extinction:
    a function of object-space points [m, 3] float32 -> [m] float32;
    majorant: the grid [D, H, W]; ray i draws from thread i of `seeds`."""
    x, w, d, hit = object_space(rays, transform)
    n = x.shape[0]
    T = np.ones(n, F)
    st = RNG.spawn(seeds, np.arange(n))
    for _ in range(rng_skip):
        st = RNG.step(st)
    alive = hit.copy()
    ds = F(density_scale)
    for _ in range(1024):
        alive &= d > 0
        ii = np.nonzero(alive)[0]
        if ii.size == 0:
            break
        mj, dist = voxel_majorant(majorant, x[ii], w[ii])
        mj = np.maximum(mj, F(1e-12))
        dist = np.maximum(dist, F(1e-6))
        u, st[ii] = RNG.uniform(st[ii])
        with np.errstate(divide="ignore"):
            ff = (-np.log((F(1) - u).astype(F)).astype(F) / (mj * ds).astype(F)).astype(F)
        dt = np.minimum(dist, ff)
        d[ii] = (d[ii] - dt).astype(F)
        x[ii] = (x[ii] + (dt[:, None] * w[ii]).astype(F)).astype(F)
        flight = dt < dist              # collided inside the voxel ...
        out_box = flight & (d[ii] <= 0)  # ... but past the box: the loop breaks
        alive[ii[out_box]] = False
        coll = flight & ~out_box
        jj = ii[coll]
        if jj.size == 0:
            continue
        sigma = np.asarray(extinction(x[jj]), F).reshape(-1)
        T[jj] = (T[jj] * (F(1) - (sigma / mj[coll]).astype(F))).astype(F)
        rr = T[jj] < F(0.05)
        kk = jj[rr]
        if kk.size:
            u2, st[kk] = RNG.uniform(st[kk])
            kill = u2 >= T[kk]
            T[kk[kill]] = 0
            alive[kk[kill]] = False
            T[kk[~kill]] = 1
    return T


def mlp_extinction(layers, head: str = "none"):
    """An extinction function for ratiotracking(): the LinearFast chain (fp16
    arithmetic, ReLU hidden layers, `head` on the last)."""
    acts = ["relu"] * (len(layers) - 1) + [head]

    def f(p):
        return field_eval(np.asarray(p, F), layers, acts)[:, 0].astype(F)
    return f
