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
  * VolumeProfile (domain/volumes.py:503-550, shaders/volumes/volume_profile.h:1-167):
    see volume_profile() below.
All arithmetic in float32, each operation rounded on its own, vectorised over
rays (every live ray runs one loop iteration per pass, so `safety` is the pass
number); VolumeProfile runs one ray at a time.
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


def mlp_extinction(layers, head: str = "none", precs=None):
    """An extinction function for ratiotracking(): the chain with each layer's
    arithmetic (precs: 'f16' LinearFast, 'f32' Linear; all 'f16' by default),
    ReLU hidden layers, `head` on the last."""
    acts = ["relu"] * (len(layers) - 1) + [head]

    def f(p):
        return field_eval(np.asarray(p, F), layers, acts, precs)[:, 0].astype(F)
    return f


# ----------------------------------------------------------------- VolumeProfile
# Reference: domain/volumes.py:503-550, shaders/volumes/volume_profile.h:1-167 (the
# active forward; the commented-out variant below it is not compiled), with
# raymarching_transmittance_trait.h, ratiotracking_transmittance_trait.h,
# random_library.h:224-239 (hg_phase_sample), math_library.h:48-57 (the slab
# test) and :323-330 (create_ortho_basis).  One ray at a time, every operation
# rounded to float32 in the shader's order; the fixed-step marches evaluate
# their extinction samples in one batch per ray.

def _f32(v) -> np.float32:
    return np.float32(v)


def _mat_vec(L: np.ndarray, v) -> np.ndarray:
    """L [3, 3] float32 times v [3]: L[i,0] v0 + L[i,1] v1 + L[i,2] v2, left to right."""
    v = np.asarray(v, F)
    return np.array([_f32(_f32(_f32(L[i, 0] * v[0]) + _f32(L[i, 1] * v[1])) + _f32(L[i, 2] * v[2]))
                     for i in range(3)], F)


def _point(x: np.ndarray, w: np.ndarray, t) -> np.ndarray:
    return (x + (w * _f32(t)).astype(F)).astype(F)


def _box(x: np.ndarray, w: np.ndarray) -> tuple[np.float32, np.float32]:
    tn, tx = ray_box32(x[None, :], w[None, :])
    return _f32(tn[0]), _f32(tx[0])


def _majorant(grid, x: np.ndarray, w: np.ndarray) -> tuple[np.float32, np.float32]:
    m, d = voxel_majorant(grid, x[None, :], w[None, :])
    return _f32(m[0]), _f32(d[0])


def crossing_tau(scale, tau) -> np.float32:
    """Expected tau at the crossing of a transmittance threshold (volume_profile.h:82)."""
    scale, tau = _f32(scale), _f32(tau)
    st = _f32(scale * tau)
    if st < _f32(0.01):
        return _f32(_f32(_f32(0.5) * scale) * tau)
    if st > _f32(20):
        return _f32(1)
    e = _f32(np.exp(_f32(-scale * tau)))
    return _f32(_f32(1) - _f32(_f32(st * e) / _f32(_f32(1) - e)))


def ortho_basis(n) -> tuple[np.ndarray, np.ndarray]:
    """math_library.h:323-330 (float32)."""
    n = np.asarray(n, F)
    sg = _f32(1) if n[2] >= 0 else _f32(-1)
    a = _f32(_f32(-1) / _f32(sg + n[2]))
    b = _f32(_f32(n[0] * n[1]) * a)
    t0 = np.array([_f32(_f32(1) + _f32(_f32(_f32(sg * n[0]) * n[0]) * a)), _f32(sg * b), _f32(-sg * n[0])], F)
    t1 = np.array([b, _f32(sg + _f32(_f32(n[1] * n[1]) * a)), _f32(-n[1])], F)
    return t0, t1


def hg_sample(w, g, st: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(direction, new state) of hg_phase_sample (random_library.h:224-239):
    the azimuth draw, then xi."""
    u, st = RNG.uniform(st)
    phi = _f32(_f32(u[0] * _f32(2)) * _f32(np.pi))
    u, st = RNG.uniform(st)
    xi = _f32(u[0])
    g = _f32(g)
    g2 = _f32(g * g)
    omg2, opg2 = _f32(_f32(1) - g2), _f32(_f32(1) + g2)
    with np.errstate(divide="ignore", invalid="ignore"):
        o2g = _f32(_f32(0.5) / g)
        t = _f32(omg2 / _f32(_f32(_f32(1) - g) + _f32(_f32(_f32(2) * g) * xi)))
        inv = _f32(o2g * _f32(opg2 - _f32(t * t)))
    ct = _f32(_f32(_f32(2) * xi) - _f32(1)) if abs(g) < _f32(0.001) else inv
    stt = _f32(np.sqrt(max(_f32(0), _f32(_f32(1) - _f32(ct * ct)))))
    t0, t1 = ortho_basis(w)
    a, b = _f32(stt * _f32(np.sin(phi))), _f32(stt * _f32(np.cos(phi)))
    w = np.asarray(w, F)
    d = np.array([_f32(_f32(_f32(a * t0[i]) + _f32(b * t1[i])) + _f32(ct * w[i])) for i in range(3)], F)
    return d, st


def _rt(grid, extinction, p, dl, d, dens, st) -> tuple[np.float32, np.ndarray]:
    """transmittance_rt (ratiotracking_transmittance_trait.h) of one ray: (T, new state)."""
    T = _f32(1)
    p = p.copy()
    d = _f32(d)
    for _ in range(1024):
        if not d > 0:
            break
        mj, dist = _majorant(grid, p, dl)
        mj = max(mj, _f32(1e-12))
        dist = max(dist, _f32(1e-6))
        u, st = RNG.uniform(st)
        with np.errstate(divide="ignore"):
            ff = _f32(_f32(-_f32(np.log(_f32(_f32(1) - u[0])))) / _f32(mj * _f32(dens)))
        dt = min(dist, ff)
        d = _f32(d - dt)
        p = (p + (dl * dt).astype(F)).astype(F)
        if dt >= dist:
            continue
        if d <= 0:
            break
        sigma = _f32(np.asarray(extinction(p[None, :]), F).reshape(-1)[0])
        T = _f32(T * _f32(_f32(1) - _f32(sigma / mj)))
        if T < _f32(0.05):
            u, st = RNG.uniform(st)
            if u[0] >= T:
                return _f32(0), st
            T = _f32(1)
    return T, st


# Steps of one fixed-step march at most (the HIP kernel's bound: the shader's
# march would not end if step_size fell below the fp32 spacing near t; for rays
# inside the box any step_size above ~1e-6 stays below it).
MAX_MARCH = 1 << 22


def _march_ts(t0, tmax, step, cap: int) -> np.ndarray:
    """t0, t0 + step, ... (each sum rounded to float32) while t < tmax, at most cap values."""
    ts = []
    t = _f32(t0)
    step = _f32(step)
    while t < tmax and len(ts) < cap:
        ts.append(t)
        t = _f32(t + step)
    return np.array(ts, F)


def dda_march_ts(x, wo, tmin, tmax, step, grid: np.ndarray, cap: int = MAX_MARCH) -> np.ndarray:
    """The sample positions t of VolumeProfileDDA's fixed-step marches
    (shaders/volumes/volume_profile_dda.h:25-77): an Amanatides-Woo walk of
    grid [D, H, W] over the box from the cell of x + wo tmin (clamped into the
    grid); in a cell whose value is > 0, t, t + step, ... while t < the cell's
    exit (= min of the three axis boundaries and tmax); then t = the exit and
    the walk steps along the axis whose boundary comes first (x, then y, then
    z on ties).  At most 4096 cells, while t < tmax, until the walk leaves the
    grid; at most cap samples (the HIP kernel's bound).  An axis whose direction
    component is 0 never comes first (+inf boundary distance and increment: the
    shader's stated intent; its arithmetic gives -inf there, and its march would
    not end).  Every operation is rounded to float32 on its own."""
    grid = np.asarray(grid, F)
    D, H, W = grid.shape[:3]
    dim = [W, H, D]
    x = np.asarray(x, F)
    wo = np.asarray(wo, F)
    tmin, tmax, step = _f32(tmin), _f32(tmax), _f32(step)
    entry = _point(x, wo, tmin)
    cell, dstep, tma, tdl = [0, 0, 0], [0, 0, 0], [F(0)] * 3, [F(0)] * 3
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        for i in range(3):
            fd = _f32(dim[i])
            cs = _f32(_f32(2) / fd)
            ci = int(np.floor(_f32(_f32(_f32(entry[i] * _f32(0.5)) + _f32(0.5)) * fd)))
            cell[i] = min(max(ci, 0), dim[i] - 1)
            dstep[i] = 1 if wo[i] > 0 else (-1 if wo[i] < 0 else 0)
            inv = _f32(_f32(1) / wo[i])
            nb = _f32(_f32(_f32(_f32(cell[i]) + _f32(max(dstep[i], 0))) * cs) - _f32(1))
            if wo[i] == 0:  # never the first axis (the shader's stated intent; its arithmetic can give -inf)
                tma[i], tdl[i] = F(np.inf), F(np.inf)
            else:
                tma[i] = _f32(_f32(nb - x[i]) * inv)
                tdl[i] = _f32(cs * _f32(abs(inv)))
        ts = []
        t = tmin
        for _ in range(4096):
            if not t < tmax:
                break
            cexit = np.fmin(np.fmin(tma[0], tma[1]), np.fmin(tma[2], tmax))
            if grid[cell[2], cell[1], cell[0]] > 0:
                while t < cexit:
                    if len(ts) >= cap:
                        return np.array(ts, F)
                    ts.append(t)
                    t = _f32(t + step)
            t = cexit
            ax = 0 if (tma[0] <= tma[1] and tma[0] <= tma[2]) else (1 if tma[1] <= tma[2] else 2)
            cell[ax] += dstep[ax]
            tma[ax] = _f32(tma[ax] + tdl[ax])
            if min(cell) < 0 or cell[0] >= W or cell[1] >= H or cell[2] >= D:
                break
    return np.array(ts, F)


def volume_profile(rays: np.ndarray, extinction, majorant: np.ndarray, seeds, thresholds, spectral_dim: int,
                   environment_samples: int = 4, g: float = 0.0, step_size: float = 0.001,
                   density_scale: float = 1.0, transform=None, light_direction=(0.0, 1.0, 0.0),
                   light_intensity=None, sample_index: int = 0, rng_skip: int = 0, albedo=None,
                   environment=None, dda_grid: np.ndarray | None = None) -> dict:
    """VolumeProfile of rays [n, 6].  extinction: object-space points [m, 3] ->
    [m] float32; majorant: the voxel grid [D, H, W]; albedo / environment:
    [m, 3] -> [m, SD] float32 (sample positions in object space, directions in
    world space).  Returns {"out": [n, DS + 3 SD + 4], "spos": [n, 3],
    "dirs": [n, ES, 3], "wts": [n, ES], "valid": [n]} (the first stage's records
    are zero where a ray does not reach them).  dda_grid [D, H, W]: VolumeProfileDDA
    (volumes.py:560-603): no end trimming, both marches at dda_march_ts's positions."""
    rays = np.asarray(rays, F).reshape(-1, 6)
    n = rays.shape[0]
    DS, SD, ES = len(thresholds), int(spectral_dim), int(environment_samples)
    OUTW = 4 + 3 * SD + DS
    thr = [_f32(v) for v in thresholds]
    intensity = [1.0] * SD if light_intensity is None else list(light_intensity)
    Mt = np.eye(4, 3, dtype=np.float64) if transform is None else np.asarray(transform, np.float64).reshape(4, 3)
    L = np.linalg.inv(Mt[0:3].T).astype(F)
    O = Mt[3].astype(F)
    ldo = _mat_vec(L, light_direction)
    step, ds, gg = _f32(step_size), _f32(density_scale), _f32(g)
    nee_ds = _f32(_f32(_f32(0.2) + _f32(_f32(0.8) * _f32(_f32(1) - gg))) * ds)
    out = np.zeros((n, OUTW), F)
    spos = np.zeros((n, 3), F)
    dirs = np.zeros((n, ES, 3), F)
    wts = np.zeros((n, ES), F)
    valid = np.zeros(n, np.int32)
    states = RNG.spawn(seeds, np.arange(n))
    for _ in range(rng_skip):
        states = RNG.step(states)

    def sig(points: np.ndarray) -> np.ndarray:
        if points.shape[0] == 0:
            return np.zeros(0, F)
        return np.asarray(extinction(points), F).reshape(-1)

    for i in range(n):
        st = states[i:i + 1]
        o = out[i]
        x = _mat_vec(L, (rays[i, 0:3] - O).astype(F))
        wo = _mat_vec(L, rays[i, 3:6])
        ww = rays[i, 3:6].copy()
        tmin, tmax = _box(x, wo)
        tmin = max(_f32(0), tmin)
        if not (tmax > 0 and tmin <= tmax):
            continue
        for _ in range(0 if dda_grid is not None else 4096):
            if not tmin < tmax:
                break
            mj, dist = _majorant(majorant, _point(x, wo, tmin), wo)
            if mj > 0:
                break
            tmin = _f32(tmin + max(dist, _f32(1e-5)))
        for _ in range(0 if dda_grid is not None else 4096):
            if not tmin < tmax:
                break
            mj, dist = _majorant(majorant, _point(x, wo, tmax), (-wo).astype(F))
            if mj > 0:
                break
            tmax = _f32(tmax - max(dist, _f32(1e-5)))
        # tau march (every sample up to tmax, then cut at the first tau > 20)
        if dda_grid is not None:
            ts = dda_march_ts(x, wo, tmin, tmax, step, dda_grid)
        else:
            ts = _march_ts(tmin, tmax, step, MAX_MARCH)
        sg = sig((x[None, :] + (wo[None, :] * ts[:, None]).astype(F)).astype(F))
        tau = _f32(0)
        for k in range(ts.size):
            tau = _f32(tau + _f32(_f32(sg[k] * ds) * step))
            if tau > _f32(20):
                break
        # depth march
        idx = 0
        scale = thr[0]
        tcross = crossing_tau(scale, tau)
        if tau > _f32(0.0001):
            ctau = _f32(0)
            for k in range(ts.size):  # the same positions as the tau march
                t = ts[k]
                ctau = _f32(ctau + _f32(_f32(sg[k] * ds) * step))
                while _f32(ctau * scale) >= tcross:
                    o[idx] = t
                    idx += 1
                    if idx >= DS:
                        break
                    scale = thr[idx]
                    tcross = crossing_tau(scale, tau)
                if idx >= DS or ctau > _f32(20):
                    break
        S = _f32(_f32(1) - _f32(np.exp(_f32(-tau))))
        o[OUTW - 1] = S
        if idx <= 0:
            continue
        check_t = o[sample_index]
        with np.errstate(invalid="ignore"):
            for k in range(DS - 1, 0, -1):
                o[k] = _f32(_f32(1) / _f32(_f32(1) + _f32(_f32(10) * _f32(np.sqrt(_f32(o[k] - o[k - 1]))))))
        o[0] = _f32(_f32(1) / _f32(_f32(0.1) + o[0]))
        sp = _point(x, wo, check_t)
        spos[i] = sp
        o[DS] = _f32(_f32(0.2) * _f32(np.log(_f32(_f32(1) + tau))))
        tn, tx = _box(sp, ldo)
        if tx < 0 or tx < tn:
            nee = _f32(1)
        else:  # transmittance_rm along the light direction: its positions, then their extinctions
            p = sp.copy()
            d = tx
            pts = []
            while d > 0 and len(pts) < 4096:
                pts.append(p)
                d = _f32(d - step)
                p = (p + (ldo * step).astype(F)).astype(F)
            sl = sig(np.array(pts, F).reshape(-1, 3))
            tl = _f32(0)
            nee = None
            for s_ in sl:
                tl = _f32(tl + _f32(_f32(s_ * nee_ds) * step))
                if tl > _f32(16):
                    nee = _f32(0)
                    break
            if nee is None:
                nee = _f32(np.exp(_f32(-tl)))
        o[DS + 1] = _f32(S * nee)
        for s in range(ES):
            dr, st = hg_sample(ww, gg, st)
            dirs[i, s] = dr
            dl = _mat_vec(L, dr)
            tn, tx = _box(sp, dl)
            T, st = _rt(majorant, extinction, sp, dl, tx, nee_ds, st)
            wts[i, s] = _f32(S * T)
        o[DS + 2 + 2 * SD] = gg
        for c in range(SD):
            o[DS + 3 + 2 * SD + c] = _f32(intensity[c])
        valid[i] = 1
    # second stage: the environment and albedo maps at the recorded directions / positions
    vi = np.nonzero(valid)[0]
    if vi.size and (albedo is not None or environment is not None):
        sa = np.asarray(albedo(spos[vi]), F).reshape(vi.size, SD) if albedo is not None else None
        env = (np.asarray(environment(dirs[vi].reshape(-1, 3)), F).reshape(vi.size, ES, SD)
               if environment is not None and ES > 0 else None)
        for j, i in enumerate(vi):
            for c in range(SD):
                if env is not None:
                    acc = _f32(0)
                    for s in range(ES):
                        acc = _f32(acc + _f32(_f32(wts[i, s] * env[j, s, c]) / _f32(ES)))
                    out[i, DS + 2 + c] = acc
                if sa is not None:
                    out[i, DS + 2 + SD + c] = _f32(_f32(1) / _f32(_f32(1) - _f32(np.log(_f32(_f32(1) - sa[j, c])))))
    return {"out": out, "spos": spos, "dirs": dirs, "wts": wts, "valid": valid}
