// VolumeProfile: per-ray features for a learned renderer (depths at transmittance
// thresholds, the light ray's transmittance, environment next-event estimates),
// with the extinction chain on the matrix cores.
#include "volume_common.h"

// RDV_FIELD_PART: 0 (this file) everything except the 8-tile instantiations
// of volume_profile_kernel and every instantiation of volume_profile_dda_kernel;
// 1 (volume_profile8.hip) the former's 8-tile launcher; 2 and 3
// (volume_profile_dda{,8}.hip) the DDA kernel's launchers: each in a
// translation unit of its own (they take most of the compile time).
#ifndef RDV_FIELD_PART
#define RDV_FIELD_PART 0
#endif

namespace rdv {

// ------------------------------------------------------------ volume profile
// VolumeProfile (src/rdv/domain/volumes.py:503-550, shaders/volumes/volume_profile.h:1-167):
// per ray, in the object space of the transform,
//   [tMin, tMax] = box interval, tMin = max(0, tMin); miss -> every output 0
//   trim both ends while the voxel majorant is 0 (steps of max(distance, 1e-5), at most 4096 each)
//   tau: t = tMin; while t < tMax: tau += sigma(x + wo t) * ds * step; t += step; stop past 20
//   depths: t = tMin again; ctau accumulates the same way; each time ctau * scale_i reaches the
//     expected crossing tau of threshold i, depth i = t; stop past 20 or after the last threshold
//   S = 1 - exp(-tau); with at least one depth: the depths re-encoded, the light ray's
//   raymarched transmittance from the sample depth's position, and per environment sample a
//   Henyey-Greenstein direction with its ratio-tracked transmittance.
// Every fp32 update is rounded on its own (no contraction), in the shader's operation order.
//
// VolumeProfileDDA (volumes.py:560-603, shaders/volumes/volume_profile_dda.h:1-208): the same,
// except that the two fixed-step marches neither trim the ends nor use the majorant field:
// they walk `majorant_grid` (a separate [D, H, W] grid over the box) cell by cell with an
// Amanatides-Woo DDA from the entry cell (at most 4096 cells, until tMax or off the grid).
// In a cell whose value is > 0 the march samples t, t + step, ... while t < the cell's exit;
// then t jumps to the exit (empty cells are skipped whole).  The light ray and the
// environment rays are VolumeProfile's.
//
// Mapping: as the ratio-tracking kernel, a wave holds 32 rays (lanes l and l + 32 mirror ray
// l); each lane runs its ray's state machine until it needs an extinction value, then the
// wave evaluates the extinction chain once for the 32 pending points.  The environment and
// albedo maps are evaluated afterwards over the recorded directions and positions
// (rdv_volume_profile_finish combines them).
struct VpArgs {
  const float* rays;
  int64_t nrays;
  const float* majorant;
  int mw, mh, md;
  float M[12];
  float density_scale, g, step;
  float light[3];
  float intensity[RDV_VP_MAX_SPECTRAL];
  float thr[RDV_VP_MAX_DEPTH];
  int ds, sd, sample_index, es;
  uint32_t seeds[4];
  int rng_skip;
  float* out;         // [n, 4 + 3 sd + ds]
  float* spos;        // [n, 3]
  float* env_dirs;    // [n, es, 3]
  float* env_w;       // [n, es]
  int32_t* valid;     // [n]
  const float* dgrid; // VolumeProfileDDA: the walked grid [dd, dh, dw] (null: VolumeProfile)
  int dw, dh, dd;
};

enum : int { kVpDone = 0, kVpTau = 1, kVpDepth = 2, kVpRm = 3, kVpRt = 4, kVpTauDda = 5, kVpDepthDda = 6 };

// Steps of one fixed-step march at most.  The shader's marches stop only at
// tMax (or tau > 20); a step below the spacing of fp32 values near t would
// never reach it, so the marches here stop after this many steps.  Between
// the box's entry and exit a march takes ceil(L / step_size) <= 3.47 / step_size
// steps, so this bound only matters below step_size ~ 1e-6.
constexpr int kVpMaxMarch = 1 << 22;

struct VpRay {
  float x[3], wo[3], ww[3];  // object-space origin and direction, world direction
  float tmin, tmax, t, tau, ctau, scale, tcross, S;
  float sp[3];               // the sample position (object space)
  float p[3], dl[3], d, T, maj;  // the secondary ray: position, direction, distance left, T or tau, majorant
  int idx, phase, k, s;
  RngState st;
  // The DDA walk (VolumeProfileDDA) during the two marches, when the secondary ray's p, dl and
  // d are free: p holds the distance to each axis' next cell boundary, dl its increment, d the
  // current cell's exit; cell the current cell; walk = cells walked, + kVpInner while t is
  // inside a marched cell.
  int cell[3];
  int walk;
};

constexpr int kVpInner = 1 << 20;  // walk flag: t is inside a marched cell (cells walked stay < 4097)

// The DDA step sign of axis i.
__device__ __forceinline__ int vp_sign(float w) { return w > 0.0f ? 1 : (w < 0.0f ? -1 : 0); }

// Expected tau at the crossing of a transmittance threshold (volume_profile.h:82).
__device__ __forceinline__ float vp_crossing(float scale, float tau) {
#pragma clang fp contract(off)
  const float st = scale * tau;
  if (st < 0.01f) return 0.5f * scale * tau;
  if (st > 20.0f) return 1.0f;
  const float e = expf(-scale * tau);
  return 1.0f - (st * e) / (1.0f - e);
}

// math_library.h:323-330: an orthonormal basis (t0, t1) around the unit vector n.
__device__ __forceinline__ void vp_basis(const float (&n)[3], float (&t0)[3], float (&t1)[3]) {
#pragma clang fp contract(off)
  const float sg = n[2] >= 0.0f ? 1.0f : -1.0f;
  const float a = -1.0f / (sg + n[2]);
  const float b = n[0] * n[1] * a;
  t0[0] = 1.0f + sg * n[0] * n[0] * a;
  t0[1] = sg * b;
  t0[2] = -sg * n[0];
  t1[0] = b;
  t1[1] = sg + n[1] * n[1] * a;
  t1[2] = -n[1];
}

// random_library.h:224-239: a direction around w distributed by the Henyey-Greenstein
// phase function with anisotropy g (two random() draws: the azimuth, then xi).
__device__ __forceinline__ void vp_hg_sample(const float (&w)[3], float g, RngState& st, float (&out)[3]) {
#pragma clang fp contract(off)
  const float phi = rng_uniform(st) * 2.0f * 3.14159265358979323846f;
  const float xi = rng_uniform(st);
  const float g2 = g * g;
  const float omg2 = 1.0f - g2, opg2 = 1.0f + g2;
  const float o2g = 0.5f / g;
  const float t = omg2 / (1.0f - g + 2.0f * g * xi);
  const float inv = o2g * (opg2 - t * t);
  const float ct = fabsf(g) < 0.001f ? 2.0f * xi - 1.0f : inv;
  const float stt = sqrtf(fmaxf(0.0f, 1.0f - ct * ct));
  float t0[3], t1[3];
  vp_basis(w, t0, t1);
  const float a = stt * sinf(phi), b = stt * cosf(phi);
#pragma unroll
  for (int i = 0; i < 3; ++i) out[i] = a * t0[i] + b * t1[i] + ct * w[i];
}

__device__ __forceinline__ void vp_point(const float (&x)[3], const float (&w)[3], float t, float (&q)[3]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 3; ++i) q[i] = x[i] + w[i] * t;
}

__device__ __forceinline__ void vp_mul3(const float (&L)[9], const float (&v)[3], float (&o)[3]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < 3; ++i) o[i] = L[i] * v[0] + L[3 + i] * v[1] + L[6 + i] * v[2];  // L column-major
}

struct VpCtx {
  const VpArgs& a;
  const float (&L)[9];
  const float (&ldo)[3];  // the light direction in object space
  float nee_ds;           // (0.2 + 0.8 (1 - g)) * density_scale
  int outw;
};

// A ray without a sample: valid 0, and zeros where the albedo and environment
// maps would read its sample position and directions, so those maps never see
// uninitialised workspace memory.
__device__ __forceinline__ void vp_invalid(const VpArgs& a, int64_t ray) {
  a.valid[ray] = 0;
  float* sp = a.spos + ray * 3;
  sp[0] = sp[1] = sp[2] = 0.0f;
  float* ed = a.env_dirs + ray * a.es * 3;
  for (int i = 0; i < 3 * a.es; ++i) ed[i] = 0.0f;
}

// The next environment sample's set-up, or the ray's last outputs after the last one.
__device__ __forceinline__ void vp_env_next(const VpCtx& c, VpRay& r, int64_t ray) {
  const VpArgs& a = c.a;
  if (r.s >= a.es) {
    float* o = a.out + ray * c.outw;
    o[a.ds + 2 + 2 * a.sd] = a.g;
    for (int i = 0; i < a.sd; ++i) o[a.ds + 3 + 2 * a.sd + i] = a.intensity[i];
    a.valid[ray] = 1;
    r.phase = kVpDone;
    return;
  }
  float dir[3];
  vp_hg_sample(r.ww, a.g, r.st, dir);
  float* ed = a.env_dirs + (ray * a.es + r.s) * 3;
  ed[0] = dir[0];
  ed[1] = dir[1];
  ed[2] = dir[2];
  vp_mul3(c.L, dir, r.dl);
  float tn, tx;
  ray_box(r.sp, r.dl, tn, tx);
#pragma unroll
  for (int i = 0; i < 3; ++i) r.p[i] = r.sp[i];
  r.d = tx;
  r.T = 1.0f;
  r.k = 0;
  r.phase = kVpRt;
}

// After the depth march (volume_profile.h:100-126).
__device__ __forceinline__ void vp_after_depth(const VpCtx& c, VpRay& r, int64_t ray) {
#pragma clang fp contract(off)
  const VpArgs& a = c.a;
  float* o = a.out + ray * c.outw;
  r.S = 1.0f - expf(-r.tau);
  o[c.outw - 1] = r.S;
  if (r.idx <= 0) {
    vp_invalid(a, ray);
    r.phase = kVpDone;
    return;
  }
  const float check_t = o[a.sample_index];
  // pow(x, 0.5) is sqrt(x) (NaN below 0, as pow is undefined there)
  for (int i = a.ds - 1; i >= 1; --i) o[i] = 1.0f / (1.0f + 10.0f * sqrtf(o[i] - o[i - 1]));
  o[0] = 1.0f / (0.1f + o[0]);
  vp_point(r.x, r.wo, check_t, r.sp);
  float* sp = a.spos + ray * 3;
  sp[0] = r.sp[0];
  sp[1] = r.sp[1];
  sp[2] = r.sp[2];
  o[a.ds] = 0.2f * logf(1.0f + r.tau);
  float tn, tx;
  ray_box(r.sp, c.ldo, tn, tx);
  if (tx < 0.0f || tx < tn) {
    o[a.ds + 1] = r.S * 1.0f;
    r.s = 0;
    vp_env_next(c, r, ray);
    return;
  }
#pragma unroll
  for (int i = 0; i < 3; ++i) r.p[i] = r.sp[i];
  r.d = tx;
  r.T = 0.0f;  // the light ray's tau
  r.k = 0;
  r.phase = kVpRm;
}

// The DDA walk's start at tmin (volume_profile_dda.h:25-51): the entry cell (clamped into
// the grid), the step signs, the distances to each axis' next cell boundary and their
// increments.  An axis whose direction component is 0 gets +inf for both, so it never comes
// first, as the shader's comment intends: its arithmetic, (boundary - x) * (1 / +0), gives
// -inf when x lies above the cell's lower boundary, and the walk would then stay at
// t = -inf (the shader's loop would not end).
__device__ __forceinline__ void vp_dda_setup(const VpCtx& c, VpRay& r) {
#pragma clang fp contract(off)
  const VpArgs& a = c.a;
  const int dim[3] = {a.dw, a.dh, a.dd};
  float entry[3];
  vp_point(r.x, r.wo, r.tmin, entry);
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const float fd = float(dim[i]);
    const float cs = 2.0f / fd;
    const int ci = int(floorf((entry[i] * 0.5f + 0.5f) * fd));
    r.cell[i] = ci < 0 ? 0 : (ci > dim[i] - 1 ? dim[i] - 1 : ci);
    const float inv = 1.0f / r.wo[i];
    const float nb = (float(r.cell[i]) + fmaxf(float(vp_sign(r.wo[i])), 0.0f)) * cs - 1.0f;
    const bool still = r.wo[i] == 0.0f;
    r.p[i] = still ? __builtin_huge_valf() : (nb - r.x[i]) * inv;
    r.dl[i] = still ? __builtin_huge_valf() : cs * fabsf(inv);
  }
  r.t = r.tmin;
  r.walk = 0;
}

// Leaves the current cell (volume_profile_dda.h:68-76): t to its exit, the next cell along
// the axis whose boundary comes first; false once the walk is off the grid.
__device__ __forceinline__ bool vp_dda_next(const VpCtx& c, VpRay& r) {
#pragma clang fp contract(off)
  r.t = r.d;
  // constant indices only: a run-time index would put the ray's state in scratch memory
  if (r.p[0] <= r.p[1] && r.p[0] <= r.p[2]) {
    r.cell[0] += vp_sign(r.wo[0]);
    r.p[0] = r.p[0] + r.dl[0];
  } else if (r.p[1] <= r.p[2]) {
    r.cell[1] += vp_sign(r.wo[1]);
    r.p[1] = r.p[1] + r.dl[1];
  } else {
    r.cell[2] += vp_sign(r.wo[2]);
    r.p[2] = r.p[2] + r.dl[2];
  }
  r.walk = (r.walk & ~kVpInner) + 1;
  return r.cell[0] >= 0 && r.cell[1] >= 0 && r.cell[2] >= 0 && r.cell[0] < c.a.dw && r.cell[1] < c.a.dh &&
         r.cell[2] < c.a.dd;
}

// Walks to the next sample point of a DDA march (true, the point in q) or to the walk's end
// (false): inside a marched cell while t < its exit, else into the next cell, skipping cells
// whose value is not > 0.
__device__ __forceinline__ bool vp_dda_walk(const VpCtx& c, VpRay& r, float (&q)[3]) {
#pragma clang fp contract(off)
  const VpArgs& a = c.a;
  for (;;) {
    if (r.walk & kVpInner) {
      if (r.t < r.d) {
        vp_point(r.x, r.wo, r.t, q);
        return true;
      }
      if (!vp_dda_next(c, r)) return false;
    }
    if (!((r.walk & ~kVpInner) < 4096 && r.t < r.tmax)) return false;
    r.d = fminf(fminf(r.p[0], r.p[1]), fminf(r.p[2], r.tmax));
    const float m = a.dgrid[(int64_t(r.cell[2]) * a.dh + r.cell[1]) * a.dw + r.cell[0]];
    if (m > 0.0f) r.walk |= kVpInner;
    else if (!vp_dda_next(c, r)) return false;
  }
}

// The depth march after the tau march (both variants; volume_profile.h:82-86).
template <bool DDA>
__device__ __forceinline__ void vp_depth_begin(const VpCtx& c, VpRay& r, int64_t ray) {
  r.t = r.tmin;
  r.k = 0;
  r.ctau = 0.0f;
  r.idx = 0;
  r.scale = c.a.thr[0];
  r.tcross = vp_crossing(r.scale, r.tau);
  if constexpr (DDA) {
    if (r.tau > 0.0001f) {
      vp_dda_setup(c, r);
      r.phase = kVpDepthDda;
    } else {
      vp_after_depth(c, r, ray);
    }
    return;
  }
  if (r.tau > 0.0001f && r.t < r.tmax) r.phase = kVpDepth;
  else vp_after_depth(c, r, ray);
}

// Ray `ray` from its input row to its first extinction request (or its end).
template <bool DDA>
__device__ __forceinline__ void vp_start(const VpCtx& c, VpRay& r, int64_t ray) {
#pragma clang fp contract(off)
  const VpArgs& a = c.a;
  const float* rr = a.rays + ray * 6;
  const float xw[3] = {rr[0] - a.M[9], rr[1] - a.M[10], rr[2] - a.M[11]};
  const float wv[3] = {rr[3], rr[4], rr[5]};
  vp_mul3(c.L, xw, r.x);
  vp_mul3(c.L, wv, r.wo);
#pragma unroll
  for (int i = 0; i < 3; ++i) r.ww[i] = wv[i];
  float* o = a.out + ray * c.outw;
  for (int i = 0; i < c.outw; ++i) o[i] = 0.0f;
  r.st = rng_spawn(a.seeds, int(ray));
  for (int k = 0; k < a.rng_skip; ++k) rng_step(r.st);
  float tmin, tmax;
  ray_box(r.x, r.wo, tmin, tmax);
  tmin = fmaxf(0.0f, tmin);
  if (!(tmax > 0.0f && tmin <= tmax)) {
    vp_invalid(a, ray);
    r.phase = kVpDone;
    return;
  }
  if constexpr (DDA) {  // VolumeProfileDDA: no trimming, the walk skips empty cells
    r.tmin = tmin;
    r.tmax = tmax;
    r.tau = 0.0f;
    r.k = 0;
    vp_dda_setup(c, r);
    r.phase = kVpTauDda;
    return;
  }
  // empty space at both ends: the voxel majorant is 0 up to its voxel's exit
  for (int skip = 0; skip < 4096 && tmin < tmax; ++skip) {
    float q[3], dist;
    vp_point(r.x, r.wo, tmin, q);
    if (voxel_majorant(a.majorant, a.mw, a.mh, a.md, q, r.wo, dist) > 0.0f) break;
    tmin = tmin + fmaxf(dist, 1e-5f);
  }
  const float nw[3] = {-r.wo[0], -r.wo[1], -r.wo[2]};
  for (int skip = 0; skip < 4096 && tmin < tmax; ++skip) {
    float q[3], dist;
    vp_point(r.x, r.wo, tmax, q);
    if (voxel_majorant(a.majorant, a.mw, a.mh, a.md, q, nw, dist) > 0.0f) break;
    tmax = tmax - fmaxf(dist, 1e-5f);
  }
  r.tmin = tmin;
  r.tmax = tmax;
  r.tau = 0.0f;
  r.t = tmin;
  r.k = 0;
  if (r.t < r.tmax) r.phase = kVpTau;
  else vp_depth_begin<DDA>(c, r, ray);
}

// Advances ray `ray` until it needs the extinction at a point (true, the point
// in q) or has finished (false).  has / sigma: the extinction at the point the
// previous call asked for.
template <bool DDA>
__device__ __forceinline__ bool vp_advance(const VpCtx& c, VpRay& r, int64_t ray, bool has, float sigma,
                                           float (&q)[3]) {
#pragma clang fp contract(off)
  const VpArgs& a = c.a;
  for (;;) {
    switch (r.phase) {
      case kVpTau:
        if (has) {
          has = false;
          r.tau = r.tau + (sigma * a.density_scale) * a.step;
          r.t = r.t + a.step;
          if (r.tau > 20.0f || !(r.t < r.tmax) || ++r.k >= kVpMaxMarch) {
            vp_depth_begin<DDA>(c, r, ray);
            break;
          }
        }
        vp_point(r.x, r.wo, r.t, q);
        return true;
      case kVpDepth:
        if (has) {
          has = false;
          r.ctau = r.ctau + (sigma * a.density_scale) * a.step;
          float* o = a.out + ray * c.outw;
          while (r.ctau * r.scale >= r.tcross) {
            o[r.idx] = r.t;
            ++r.idx;
            if (r.idx >= a.ds) break;
            r.scale = a.thr[r.idx];
            r.tcross = vp_crossing(r.scale, r.tau);
          }
          bool stop = r.idx >= a.ds;
          if (!stop) {
            r.t = r.t + a.step;
            stop = r.ctau > 20.0f || !(r.t < r.tmax) || ++r.k >= kVpMaxMarch;
          }
          if (stop) {
            vp_after_depth(c, r, ray);
            break;
          }
        }
        vp_point(r.x, r.wo, r.t, q);
        return true;
      case kVpTauDda:  // volume_profile_dda.h:53-77
        if constexpr (DDA) {
          if (has) {
            has = false;
            r.tau = r.tau + (sigma * a.density_scale) * a.step;
            r.t = r.t + a.step;
            if (r.tau > 20.0f || ++r.k >= kVpMaxMarch) {
              vp_depth_begin<DDA>(c, r, ray);
              break;
            }
          }
          if (vp_dda_walk(c, r, q)) return true;
          vp_depth_begin<DDA>(c, r, ray);
          break;
        } else {
          return false;
        }
      case kVpDepthDda:  // volume_profile_dda.h:83-129
        if constexpr (DDA) {
          if (has) {
            has = false;
            r.ctau = r.ctau + (sigma * a.density_scale) * a.step;
            float* o = a.out + ray * c.outw;
            while (r.ctau * r.scale >= r.tcross) {
              o[r.idx] = r.t;
              ++r.idx;
              if (r.idx >= a.ds) break;
              r.scale = a.thr[r.idx];
              r.tcross = vp_crossing(r.scale, r.tau);
            }
            bool stop = r.idx >= a.ds;
            if (!stop) {
              r.t = r.t + a.step;
              stop = r.ctau > 20.0f || ++r.k >= kVpMaxMarch;
            }
            if (stop) {
              vp_after_depth(c, r, ray);
              break;
            }
          }
          if (vp_dda_walk(c, r, q)) return true;
          vp_after_depth(c, r, ray);
          break;
        } else {
          return false;
        }
      case kVpRm:  // raymarching_transmittance_trait.h
        if (has) {
          has = false;
          r.T = r.T + (sigma * c.nee_ds) * a.step;
          if (r.T > 16.0f) {
            a.out[ray * c.outw + a.ds + 1] = r.S * 0.0f;
            r.s = 0;
            vp_env_next(c, r, ray);
            break;
          }
          r.d = r.d - a.step;
#pragma unroll
          for (int i = 0; i < 3; ++i) r.p[i] = r.p[i] + a.step * c.ldo[i];
          ++r.k;
        }
        if (!(r.d > 0.0f && r.k < 4096)) {
          a.out[ray * c.outw + a.ds + 1] = r.S * expf(-r.T);
          r.s = 0;
          vp_env_next(c, r, ray);
          break;
        }
#pragma unroll
        for (int i = 0; i < 3; ++i) q[i] = r.p[i];
        return true;
      case kVpRt: {  // ratiotracking_transmittance_trait.h
        bool end = false;
        if (has) {
          has = false;
          r.T = r.T * (1.0f - sigma / r.maj);
          if (r.T < 0.05f) {
            if (rng_uniform(r.st) >= r.T) {
              r.T = 0.0f;
              end = true;
            } else {
              r.T = 1.0f;
            }
          }
        }
        while (!end) {
          if (!(r.d > 0.0f && r.k < 1024)) break;
          float dist;
          float mj = voxel_majorant(a.majorant, a.mw, a.mh, a.md, r.p, r.dl, dist);
          mj = fmaxf(mj, 1e-12f);
          dist = fmaxf(dist, 1e-6f);
          const float u = rng_uniform(r.st);
          const float ff = -logf(1.0f - u) / (mj * c.nee_ds);
          const float dt = fminf(dist, ff);
          r.d = r.d - dt;
#pragma unroll
          for (int i = 0; i < 3; ++i) r.p[i] = r.p[i] + dt * r.dl[i];
          ++r.k;
          if (dt >= dist) continue;
          if (r.d <= 0.0f) break;
          r.maj = mj;
#pragma unroll
          for (int i = 0; i < 3; ++i) q[i] = r.p[i];
          return true;
        }
        a.env_w[ray * a.es + r.s] = r.S * r.T;
        ++r.s;
        vp_env_next(c, r, ray);
        break;
      }
      default:
        return false;
    }
  }
}

struct VpGenArgs {
  VpArgs v;
  const uint8_t* packed;
  GenNet net;
};

// One block's rays (DDA: VolumeProfileDDA's marches, a compile-time choice so that
// VolumeProfile's kernel carries none of the walk's state).  W64: 64 rays per
// wave, one per lane, with GenFieldNet evaluated for both 32-point tiles at once
// (gen_field_pair64); otherwise 32 per wave, lanes l and l + 32 carrying the same
// ray (the chain's two K halves of one MFMA column).
template <int MT, bool LDSW, bool DDA, bool F32L, bool W64 = false>
__device__ __forceinline__ void volume_profile_body(const VpGenArgs& ga) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_next;
  const VpArgs& a = ga.v;
  const GenNet& g = ga.net;
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  const bool has_bias = packed_has_bias(ga.packed);
  const half8* w0;
  const float* b0;
  gen_sources<LDSW>(ga.packed, g, smem, &w0, &b0);
  if (threadIdx.x == 0) s_next = 0;
  __syncthreads();
  const int act = g.act[g.L - 1];
  const BlockRays br(a.nrays);
  const int nr = br.count;
  float L[9];
  inverse3(a.M, L);
  float ldo[3];
  vp_mul3(L, a.light, ldo);
  float nee_ds;
  {
#pragma clang fp contract(off)
    nee_ds = (0.2f + 0.8f * (1.0f - a.g)) * a.density_scale;
  }
  const VpCtx c{a, L, ldo, nee_ds, 4 + 3 * a.sd + a.ds};

  VpRay r = {};
  int64_t ray = -1;        // the ray in this column (-1: none)
  bool pending = false;    // q is a point waiting for its extinction
  bool has = false;        // sigma holds the extinction at the last requested point
  bool exhausted = false;  // the block's range has run dry
  float q[3] = {0.0f, 0.0f, 0.0f};
  float sigma = 0.0f;
  const uint64_t below = (uint64_t(1) << (W64 ? lane : col)) - 1;
  const bool owner = W64 || h == 0;  // the lane whose ballot bit stands for its ray
  for (;;) {
    for (;;) {
      if (ray >= 0 && !pending) {
        pending = vp_advance<DDA>(c, r, ray, has, sigma, q);
        has = false;
        if (!pending) ray = -1;
      }
      const bool idle = ray < 0 && !exhausted;
      const uint64_t want = __builtin_amdgcn_ballot_w64(owner && idle);
      if (want == 0) break;
      int base = 0;
      if (lane == 0) base = atomicAdd(&s_next, __builtin_popcountll(want));
      base = __builtin_amdgcn_readfirstlane(base);
      if (idle) {  // (32 rays per wave: both halves see the same `want` bits of the h == 0 lanes)
        const int k = base + __builtin_popcountll(want & below);
        if (k < nr) {
          ray = br.ray(k);
          if (ray >= a.nrays) {
            ray = -1;  // past the last ray: claim again
          } else {
            vp_start<DDA>(c, r, ray);
            if (r.phase == kVpDone) ray = -1;
          }
        } else {
          exhausted = true;
        }
      }
    }
    if (__builtin_amdgcn_ballot_w64(owner && pending) == 0) break;  // every ray is out of work
    float p[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) p[i] = pending ? q[i] : 0.0f;
    float s;
    if constexpr (W64) {
      s = gen_field_pair64(w0, b0, has_bias, lane, h, p, act);
    } else {
      s = gen_field_row0<MT, F32L>(g, w0, b0, has_bias, lane, h, p, act);
      s = __shfl(s, col);  // the value of lane col (row 0 of its column)
    }
    if (pending) {
      sigma = s;
      has = true;
      pending = false;
    }
  }
}

template <int MT, bool LDSW, bool F32L = false>
__global__ __launch_bounds__(64 * gen_waves<MT>(), 1) void volume_profile_kernel(VpGenArgs ga) {
  volume_profile_body<MT, LDSW, false, F32L>(ga);
}

template <int MT, bool LDSW, bool F32L = false>
__global__ __launch_bounds__(64 * gen_waves<MT>(), 1) void volume_profile_dda_kernel(VpGenArgs ga) {
  volume_profile_body<MT, LDSW, true, F32L>(ga);
}

// 64 rays per wave for the chains that are GenFieldNet (GenNet::fast), weights in LDS.
template <bool DDA>
__global__ __launch_bounds__(64 * gen_waves<2>(), 1) void volume_profile64_kernel(VpGenArgs ga) {
  volume_profile_body<2, true, DDA, false, true>(ga);
}

// Launch of volume_profile64_kernel<DDA> (64 rays per wave).
template <bool DDA>
static int launch_volume_profile64(const VpGenArgs& ga, int64_t nrays, int cu, hipStream_t stream) {
  return launch_gen_field<VpGenArgs, 2, true>(&volume_profile64_kernel<DDA>, ga, (nrays + 63) / 64, cu,
                                               gen_lds_bytes(ga.net), stream);
}

// volume_profile.h:155-160 for the rows that reached a depth.
struct VpFinishArgs {
  const float* albedo;
  int64_t albedo_stride;
  const float* env;
  int64_t env_stride;
  const float* env_w;
  const int32_t* valid;
  int64_t nrays;
  int ds, sd, es;
  float* out;
};

// 8-tile launcher of volume_profile_kernel (RDV_FIELD_PART 1); every launch of
// volume_profile_dda_kernel (RDV_FIELD_PART 2) and its 8-tile launcher (RDV_FIELD_PART 3).
int launch_volume_profile8(const VpGenArgs& a, int64_t items, int cu, int64_t lds, bool in_lds, hipStream_t stream);
int launch_volume_profile_dda_any(const VpGenArgs& a, int64_t items, int cu, bool mixed, hipStream_t stream);
int launch_volume_profile_dda8(const VpGenArgs& a, int64_t items, int cu, int64_t lds, bool in_lds,
                               hipStream_t stream);

#if RDV_FIELD_PART == 0
__global__ __launch_bounds__(256) void volume_profile_finish_kernel(VpFinishArgs f) {
#pragma clang fp contract(off)
  const int outw = 4 + 3 * f.sd + f.ds;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < f.nrays; i += int64_t(gridDim.x) * blockDim.x) {
    if (f.valid[i] == 0) continue;
    float* o = f.out + i * outw;
    for (int ch = 0; ch < f.sd; ++ch) {
      float acc = 0.0f;
      for (int s = 0; s < f.es; ++s) {
        const int64_t row = i * f.es + s;
        acc = acc + f.env_w[row] * f.env[row * f.env_stride + ch] / float(f.es);
      }
      o[f.ds + 2 + ch] = acc;
      const float sa = f.albedo[i * f.albedo_stride + ch];
      o[f.ds + 2 + f.sd + ch] = 1.0f / (1.0f - logf(1.0f - sa));
    }
  }
}

int launch_volume_profile(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed,
                          const rdv_volume_profile_desc& vp, const float* majorant, const float* dda_grid, int dda_w,
                          int dda_h, int dda_d, const float* rays, int64_t nrays, float* out, float* spos,
                          float* env_dirs, float* env_w, int32_t* valid, hipStream_t stream) {
  std::string why;
  const bool mixed = is_mixed_field(d, lay, 1, &why);
  if (!mixed && !is_f16_field(d, 1))
    return fail(RDV_ERR_UNSUPPORTED, why.empty() ? "the extinction must be a chain of LinearFast / Linear layers from 3 "
                                                   "inputs to 1 output" : why);
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  VpGenArgs ga;
  VpArgs& a = ga.v;
  a.rays = rays;
  a.nrays = nrays;
  a.majorant = majorant;
  a.mw = vp.maj_width;
  a.mh = vp.maj_height;
  a.md = vp.maj_depth;
  for (int i = 0; i < 12; ++i) a.M[i] = vp.transform[i];
  a.density_scale = vp.density_scale;
  a.g = vp.g;
  a.step = vp.step_size;
  for (int i = 0; i < 3; ++i) a.light[i] = vp.light_direction[i];
  for (int i = 0; i < RDV_VP_MAX_SPECTRAL; ++i) a.intensity[i] = vp.light_intensity[i];
  for (int i = 0; i < RDV_VP_MAX_DEPTH; ++i) a.thr[i] = vp.transmittance_threshold[i];
  a.ds = vp.depth_samples;
  a.sd = vp.spectral_dim;
  a.sample_index = vp.sample_index;
  a.es = vp.environment_samples;
  for (int i = 0; i < 4; ++i) a.seeds[i] = vp.seeds[i];
  a.rng_skip = vp.rng_skip;
  a.out = out;
  a.spos = spos;
  a.env_dirs = env_dirs;
  a.env_w = env_w;
  a.valid = valid;
  a.dgrid = dda_grid;
  a.dw = dda_w;
  a.dh = dda_h;
  a.dd = dda_d;
  ga.packed = static_cast<const uint8_t*>(packed);
  gen_net(d, lay, &ga.net);
  // GenFieldNet: 64 rays per wave
  if (!mixed && ga.net.fast && gen_lds_bytes(ga.net) <= kGenFieldLdsCap)
    return dda_grid != nullptr ? launch_volume_profile64<true>(ga, nrays, di.cu_count, stream)
                               : launch_volume_profile64<false>(ga, nrays, di.cu_count, stream);
  // 32 rays per wave
  if (dda_grid != nullptr) return launch_volume_profile_dda_any(ga, (nrays + 31) / 32, di.cu_count, mixed, stream);
  if (mixed) RDV_GEN_FIELD_DISPATCH_MIXED(volume_profile_kernel, ga, (nrays + 31) / 32, di.cu_count, ga.net, stream);
  RDV_GEN_FIELD_DISPATCH(volume_profile_kernel, ga, (nrays + 31) / 32, di.cu_count, ga.net, stream,
                         launch_volume_profile8);
}

int launch_volume_profile_finish(const rdv_volume_profile_desc& vp, const float* albedo, int64_t albedo_stride,
                                 const float* env, int64_t env_stride, const float* env_w, const int32_t* valid,
                                 int64_t nrays, float* out, hipStream_t stream) {
  VpFinishArgs f{albedo, albedo_stride, env, env_stride, env_w, valid, nrays,
                 vp.depth_samples, vp.spectral_dim, vp.environment_samples, out};
  int64_t blocks = (nrays + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  volume_profile_finish_kernel<<<dim3(unsigned(blocks)), dim3(256), 0, stream>>>(f);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

#elif RDV_FIELD_PART == 1
RDV_GEN_FIELD_DEFINE8(launch_volume_profile8, volume_profile_kernel, VpGenArgs)
#elif RDV_FIELD_PART == 2
int launch_volume_profile_dda_any(const VpGenArgs& a, int64_t items, int cu, bool mixed, hipStream_t stream) {
  VpGenArgs ga = a;
  if (mixed) RDV_GEN_FIELD_DISPATCH_MIXED(volume_profile_dda_kernel, ga, items, cu, ga.net, stream);
  RDV_GEN_FIELD_DISPATCH(volume_profile_dda_kernel, ga, items, cu, ga.net, stream, launch_volume_profile_dda8);
}
#elif RDV_FIELD_PART == 3
RDV_GEN_FIELD_DEFINE8(launch_volume_profile_dda8, volume_profile_dda_kernel, VpGenArgs)
#endif  // RDV_FIELD_PART

}  // namespace rdv
