// Pinhole camera rays of the Cameras grid (src/rdv/domain/rendering.py:10-42,
// src/rdv/shaders/rendering/cameras.h:1-20), shared by the full-grid ray
// kernel, the fused renderers and the batched grid evaluation.
#pragma once

#include "rdv_common.h"

namespace rdv {

struct CameraParams {
  const float* poses;  // [n, 9]: origin, target, up
  int n, H, W;
  float aspect, fov;
};

// cameras.h: pixel centre p = ((x, y) + 0.5) / (W, H) * 2 - 1, s = (p.x * aspect,
// p.y, 1 / tan(fov / 2)), frame z = normalize(target - origin),
// x = normalize(cross(up, z)), y = cross(z, x), w = normalize(s.x x + s.y y + s.z z).
// (jx, jy) is the sub-pixel position: the centre (1/2, 1/2), or two random
// numbers for a jittered camera (cameras.h:7).
__device__ __forceinline__ void camera_ray(const CameraParams& c, int cam, int y, int x, float (&o)[3],
                                           float (&w)[3], float jx = 0.5f, float jy = 0.5f) {
  const float* P = c.poses + int64_t(cam) * 9;
  float t[3], n[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    o[i] = P[i];
    t[i] = P[3 + i];
    n[i] = P[6 + i];
  }
  const float px = (float(x) + jx) / float(c.W) * 2.0f - 1.0f;
  const float py = (float(y) + jy) / float(c.H) * 2.0f - 1.0f;
  const float sx = px * c.aspect, sy = py, sz = 1.0f / tanf(c.fov * 0.5f);
  float z[3] = {t[0] - o[0], t[1] - o[1], t[2] - o[2]};
  float inv = 1.0f / sqrtf(z[0] * z[0] + z[1] * z[1] + z[2] * z[2]);
#pragma unroll
  for (int i = 0; i < 3; ++i) z[i] *= inv;
  float xa[3] = {n[1] * z[2] - n[2] * z[1], n[2] * z[0] - n[0] * z[2], n[0] * z[1] - n[1] * z[0]};
  inv = 1.0f / sqrtf(xa[0] * xa[0] + xa[1] * xa[1] + xa[2] * xa[2]);
#pragma unroll
  for (int i = 0; i < 3; ++i) xa[i] *= inv;
  const float ya[3] = {z[1] * xa[2] - z[2] * xa[1], z[2] * xa[0] - z[0] * xa[2], z[0] * xa[1] - z[1] * xa[0]};
#pragma unroll
  for (int i = 0; i < 3; ++i) w[i] = xa[i] * sx + ya[i] * sy + z[i] * sz;
  inv = 1.0f / sqrtf(w[0] * w[0] + w[1] * w[1] + w[2] * w[2]);
#pragma unroll
  for (int i = 0; i < 3; ++i) w[i] *= inv;
}

struct JitterSeeds {
  int on;             // 0: pixel centres
  uint32_t seeds[4];  // the dispatch's random seeds
};

}  // namespace rdv
