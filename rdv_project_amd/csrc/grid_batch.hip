// Batch branch of Grid.__call__ (src/rdv/maths/__init__.py:104-119,
// src/rdv/shaders/grids/batch_grid_evaluator.h): one thread per requested index
// vector of a batch idx[n, rank] (int32, the grid's IN-sized index in its last
// dimension) instead of one per grid cell.
//
//  - cameras_rays_at_kernel: Cameras' forward at the index vectors (cam, y, x)
//    (shaders/rendering/cameras.h:1-20).  Thread i is batch row i, so a
//    jittered camera draws from thread i's generator of the dispatch, as the
//    reference's batch evaluator does.
//  - grid_gather_kernel: the rows of a grid whose values are materialised in
//    HBM ([*shape, width] fp32, row-major with the last dimension fastest:
//    grid_library.h:3-16's indices_to_global), i.e. TensorGrid's forward
//    (shaders/grids/tensor_grid.h) and every grid node that this build
//    evaluates into a buffer.
//
// An index component outside its grid dimension (the camera index outside
// [0, n_cams)) gives a row of NaN: the reference's shader reads past the
// buffer there; here nothing outside it is touched.  A camera's y and x are
// free, as in the shader's formula (a ray through a point off the image).
#include "camera.h"

namespace rdv {

__global__ __launch_bounds__(256) void cameras_rays_at_kernel(CameraParams c, JitterSeeds js,
                                                              const int32_t* __restrict__ idx, int64_t n,
                                                              float* __restrict__ rays) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const int cam = idx[3 * i], y = idx[3 * i + 1], x = idx[3 * i + 2];
    float* dst = rays + i * 6;
    if (cam < 0 || cam >= c.n) {
#pragma unroll
      for (int k = 0; k < 6; ++k) dst[k] = __builtin_nanf("");
      continue;
    }
    float jx = 0.5f, jy = 0.5f;
    if (js.on) {  // the batch evaluator's thread index is the batch row
      RngState st = rng_spawn(js.seeds, int(i));
      jx = rng_uniform(st);
      jy = rng_uniform(st);
    }
    float o[3], w[3];
    camera_ray(c, cam, y, x, o, w, jx, jy);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      dst[k] = o[k];
      dst[3 + k] = w[k];
    }
  }
}

struct GatherGrid {
  int rank, width;
  int64_t shape[RDV_GRID_MAX_RANK];
};

// One thread per output element (row e / width, component e % width): a row's
// components are consecutive threads, so both the gather and the store are
// contiguous runs of `width` floats.
__global__ __launch_bounds__(256) void grid_gather_kernel(const float* __restrict__ values, GatherGrid g,
                                                          const int32_t* __restrict__ idx, int64_t total,
                                                          float* __restrict__ out) {
  for (int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x) {
    const int64_t row = e / g.width;
    const int comp = int(e - row * g.width);
    const int32_t* v = idx + row * g.rank;
    int64_t cell = 0;
    bool inside = true;
    for (int d = 0; d < g.rank; ++d) {
      const int32_t k = v[d];
      inside = inside && k >= 0 && int64_t(k) < g.shape[d];
      cell = cell * g.shape[d] + (inside ? k : 0);
    }
    out[e] = inside ? values[cell * g.width + comp] : __builtin_nanf("");
  }
}

static int grid_blocks(int64_t total, unsigned* blocks) {
  DeviceInfo di;
  const int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  int64_t b = (total + 255) / 256;
  const int64_t cap = int64_t(di.cu_count) * 16;
  *blocks = unsigned(b < cap ? (b < 1 ? 1 : b) : cap);
  return RDV_OK;
}

int launch_cameras_rays_at(const rdv_camera_desc& c, const float* poses, const int32_t* idx, int64_t n,
                           const uint32_t* seeds, float* rays, hipStream_t stream) {
  if (n == 0) return RDV_OK;
  CameraParams p{poses, c.n_cams, c.height, c.width, c.aspect_ratio, c.fov};
  JitterSeeds js{0, {0, 0, 0, 0}};
  if (seeds != nullptr) js = JitterSeeds{1, {seeds[0], seeds[1], seeds[2], seeds[3]}};
  unsigned blocks = 0;
  if (int rc = grid_blocks(n, &blocks)) return rc;
  cameras_rays_at_kernel<<<dim3(blocks), dim3(256), 0, stream>>>(p, js, idx, n, rays);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

int launch_grid_gather(const float* values, int rank, const int64_t* shape, int width, const int32_t* idx, int64_t n,
                       float* out, hipStream_t stream) {
  if (n == 0) return RDV_OK;
  GatherGrid g;
  g.rank = rank;
  g.width = width;
  for (int d = 0; d < RDV_GRID_MAX_RANK; ++d) g.shape[d] = d < rank ? shape[d] : 1;
  unsigned blocks = 0;
  if (int rc = grid_blocks(n * width, &blocks)) return rc;
  grid_gather_kernel<<<dim3(blocks), dim3(256), 0, stream>>>(values, g, idx, n * width, out);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

}  // namespace rdv
