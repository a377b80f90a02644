// Camera rays, MLP-in-the-loop volume rendering and compositing.
//
//  - camera_rays_kernel: Cameras (src/rdv/domain/rendering.py:10-42,
//    src/rdv/shaders/rendering/cameras.h:1-20), one thread per (cam, y, x).
//  - render_ea_kernel: build-defined emission-absorption renderer of the
//    benchmark configuration: per pixel ray through the box [-1,1]^3, S samples
//    t_i = t0 + (i + 1/2) dt, dt = (t1 - t0) / S, each fed through the fused
//    fp16 MLP (density / RGB head), composited front to back in fp32:
//    alpha_i = 1 - exp(-sigma_i dt), T_i = prod_{j<i} (1 - alpha_j),
//    C = sum_i T_i alpha_i c_i.
//  - composite_kernel: the same compositing over precomputed samples
//    (sigma, r, g, b) streamed from HBM (exclusive optical depth per sample from
//    a per-lane partial sum and one wavefront scan).
//  - raymarch_transmittance_kernel: RaymarchingTransmittance
//    (src/rdv/domain/volumes.py:124-141, shaders/volumes/raymarching_transmittance.h,
//    raymarching_transmittance_trait.h, libraries/math_library.h:48-57) with
//    the extinction map evaluated on the matrix cores 32 march steps at a time.
//
// MLP-in-the-loop mapping: one wave owns one ray at a time; a 32-sample chunk
// of the ray is one MFMA N block (lane l evaluates sample l % 32, both feature
// halves), and two consecutive chunks go through the layer chain together as
// the fused MLP kernel's staggered tile pair (run_pair, mlp_core.h).  The
// samples' positions are generated in registers and the head values never
// leave the wave: transmittance along a chunk is an inclusive wavefront scan of
// sigma * dt (T_i = T_in exp(-sum_{j<i} sigma_j dt)), the chunks composited in
// ray order, the colour a per-lane partial sum reduced once per ray.
#include "camera.h"
#include "volume_common.h"

// RDV_FIELD_PART selects what this translation unit emits: 0 (render.hip
// itself) everything except the 8-tile instantiations of the runtime-shaped
// field kernels; 1, 2, 3 (render_field8_{march,ratio,ea}.hip) the 8-tile
// launcher of one of those kernels.  The 8-tile kernels take most of the
// compile time, and separate units build in parallel.
#ifndef RDV_FIELD_PART
#define RDV_FIELD_PART 0
#endif

namespace rdv {

#if RDV_FIELD_PART == 0
__global__ void camera_rays_kernel(CameraParams c, JitterSeeds js, float* __restrict__ rays) {
  const int64_t total = int64_t(c.n) * c.H * c.W;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    const int x = int(i % c.W);
    const int64_t r = i / c.W;
    const int y = int(r % c.H);
    const int cam = int(r / c.H);
    float jx = 0.5f, jy = 0.5f;
    if (js.on) {  // thread i's generator (the grid evaluator's thread index is the cell index)
      RngState st = rng_spawn(js.seeds, int(i));
      jx = rng_uniform(st);
      jy = rng_uniform(st);
    }
    float o[3], w[3];
    camera_ray(c, cam, y, x, o, w, jx, jy);
    float* dst = rays + i * 6;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      dst[k] = o[k];
      dst[3 + k] = w[k];
    }
  }
}
#endif

// ------------------------------------------------------------ wave helpers
// Inclusive prefix sum over the 64 lanes of a wave with DPP lane moves (no LDS
// traffic): shifts by 1, 2, 4, 8 inside each 16-lane row, then row 0's / 1's
// last lane broadcast into rows 1 / 3 (row_bcast:15) and lane 31 into rows 2, 3
// (row_bcast:31).  Out-of-row sources read 0 (bound_ctrl).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, true));
}
__device__ __forceinline__ float wave_scan_incl(float v, int /*lane*/) {
  v += dpp_move<0x111, 0xF>(v);  // row_shr:1
  v += dpp_move<0x112, 0xF>(v);  // row_shr:2
  v += dpp_move<0x114, 0xF>(v);  // row_shr:4
  v += dpp_move<0x118, 0xF>(v);  // row_shr:8
  v += dpp_move<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  v += dpp_move<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
  return v;
}
// Inclusive prefix sums over each 32-lane half of a wave separately: the
// first five steps of wave_scan_incl (lanes 0..31 get the same bits as from
// it, lanes 32..63 the same scan of their own half).
__device__ __forceinline__ float wave_scan_incl32(float v) {
  v += dpp_move<0x111, 0xF>(v);  // row_shr:1
  v += dpp_move<0x112, 0xF>(v);  // row_shr:2
  v += dpp_move<0x114, 0xF>(v);  // row_shr:4
  v += dpp_move<0x118, 0xF>(v);  // row_shr:8
  v += dpp_move<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  return v;
}
// Sum over the wave, returned in every lane.
__device__ __forceinline__ float wave_sum(float v) {
  const float incl = wave_scan_incl(v, 0);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, incl), 63));
}
// Value of lane `src` (wave-uniform) in every lane.
__device__ __forceinline__ float lane_value(float v, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

// The MLP of one 32-sample chunk: p is this lane's sample (lanes l and l + 32
// hold the same sample), fin the last layer's accumulators.
template <class N, bool RELU>
__device__ __forceinline__ void eval_chunk(const half8* sw, const float* sb, bool has_bias, int lane, int h,
                                           const float (&p)[N::kIn], f32x16 (&fin)[N::kMaxMT]) {
  constexpr int LL = N::kL - 1;
  f32x16 accA[N::kMaxMT], accB[N::kMaxMT];
  half8 b[N::kMaxKC];
  const LdsWeights ws{sw + opaque_zero(), lane};
  if (has_bias) {
    const float* sbt = sb + opaque_zero();
    load_bias<N, 0>(accA, sbt, h);
    build_input<N>(p, h, b);
    run_chain<N, 0, RELU, true>(ws, b, accA, accB, sbt, h);
  } else {
    build_input<N>(p, h, b);
    run_chain<N, 0, RELU, false>(ws, b, accA, accB, sb, h);
  }
#pragma unroll
  for (int t = 0; t < N::kMaxMT; ++t) fin[t] = (LL % 2 == 0) ? accA[t] : accB[t];
}

constexpr int kRenderWaves = 16;  // transmittance kernel
constexpr int kRenderThreads = 64 * kRenderWaves;
// emission-absorption renderer: 12 waves (3 per SIMD; the tile-pair chain needs
// ~168 registers), measured faster than 8 or 16
constexpr int kEaWaves = 12;
constexpr int kEaThreads = 64 * kEaWaves;

// Weights and biases of the packed MLP into LDS (block of THREADS threads), counter reset.
template <class N, int THREADS>
__device__ __forceinline__ void stage_weights(const uint8_t* packed, const MlpLayout& lay, float* sb, half8* sw,
                                              int* s_next) {
  stage_net_weights<N, THREADS>(packed, lay, sb, sw);
  if (threadIdx.x == 0) *s_next = 0;
  __syncthreads();
}

// ------------------------------------------------------ emission-absorption
struct RenderArgs {
  CameraParams cam;
  const float* rays;  // [n_rays, 6] (origin, direction) in memory, or null: the rays of `cam`
  int64_t n_rays;     // with `rays`
  const uint8_t* packed;
  MlpLayout lay;
  float* image;  // [n, H, W, 3] (or [n_rays, 3])
  int samples;   // multiple of 32
};

__device__ __forceinline__ int64_t ea_ray_count(const RenderArgs& a) {
  return a.rays != nullptr ? a.n_rays : int64_t(a.cam.n) * a.cam.H * a.cam.W;
}

// Origin and direction of ray `ray`: read from memory, or the camera's pixel ray.
__device__ __forceinline__ void ea_ray(const RenderArgs& a, int64_t ray, float (&o)[3], float (&w)[3]) {
  if (a.rays != nullptr) {
    const float* r = a.rays + ray * 6;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      o[i] = r[i];
      w[i] = r[3 + i];
    }
    return;
  }
  const int x = int(ray % a.cam.W);
  const int64_t rest = ray / a.cam.W;
  const int y = int(rest % a.cam.H);
  const int cam = int(rest / a.cam.H);
  camera_ray(a.cam, cam, y, x, o, w);
}

// A wave-uniform float moved to a scalar register (the ray's geometry and
// transmittance are the same in every lane of its wave; in SGPRs they do not
// compete with the MLP chain's VGPRs).
__device__ __forceinline__ float wave_uniform(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// The march geometry of ray `ray`: p = (origin, w.x), q = (w.y, w.z, entry
// distance, step); a step of -1 marks a ray that misses the box.
__device__ __forceinline__ void ea_setup(const RenderArgs& a, int64_t ray, f32x4& p, f32x4& q) {
  float o[3], w[3];
  ea_ray(a, ray, o, w);
  float t0, t1;
  ray_box(o, w, t0, t1);
  float dt = -1.0f;
  if (!(t1 <= 0.0f || t0 > t1)) {
    t0 = fmaxf(t0, 0.0f);
    dt = (t1 - t0) / float(a.samples);
  }
  p = f32x4{o[0], o[1], o[2], w[0]};
  q = f32x4{w[1], w[2], t0, dt};
}

// Rays whose geometry a block computes at once, one ray per thread, into LDS
// (32 bytes each): the camera frame, slab test and step are then computed once
// per ray instead of in all 64 lanes of the wave that marches it.
constexpr int kEaBatch = 2048;

template <class N>
__global__ __launch_bounds__(kEaThreads, 1) void render_ea_kernel(RenderArgs a) {
  static_assert(N::kIn == 3 && N::kOut == 4, "the renderer evaluates a 3 -> 4 (density, RGB) field");
  __shared__ float sb[N::kBias];
  __shared__ half8 sw[N::kFrags * 64];
  __shared__ f32x4 s_ray[2][kEaBatch];
  __shared__ int s_next;
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  const int64_t nrays = ea_ray_count(a);
  const BlockRays br(nrays, false);
  const int nr = br.count;
  const bool has_bias = packed_has_bias(a.packed);
  stage_weights<N, kEaThreads>(a.packed, a.lay, sb, sw, &s_next);

  auto claim = [&]() {
    int t = 0;
    if (lane == 0) t = atomicAdd(&s_next, 1);
    return __builtin_amdgcn_readfirstlane(t);
  };
  const int chunks = a.samples / 32;
  // Batches of kEaBatch rays: every thread sets up its rays, then the waves
  // claim them one by one; a barrier ends each batch (counter and ray slots
  // are reused).
  for (int base = 0; base < nr; base += kEaBatch) {
    const int nb = nr - base < kEaBatch ? nr - base : kEaBatch;
    for (int i = threadIdx.x; i < nb; i += kEaThreads) {
      const int64_t ray = br.ray(base + i);
      if (ray < nrays) {
        ea_setup(a, ray, s_ray[0][i], s_ray[1][i]);
      } else {  // past the last ray: nothing to march, nothing to write
        s_ray[0][i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        s_ray[1][i] = f32x4{0.0f, 0.0f, 0.0f, -1.0f};
      }
    }
    if (threadIdx.x == 0) s_next = 0;
    __syncthreads();
    for (int r = claim(); r < nb; r = claim()) {
      const int64_t ray = br.ray(base + r);
      const f32x4 p4 = s_ray[0][r], q4 = s_ray[1][r];
      const float o[3] = {wave_uniform(p4[0]), wave_uniform(p4[1]), wave_uniform(p4[2])};
      const float w[3] = {wave_uniform(p4[3]), wave_uniform(q4[0]), wave_uniform(q4[1])};
      const float t0 = wave_uniform(q4[2]), dt = wave_uniform(q4[3]);
      float cr = 0.0f, cg = 0.0f, cb = 0.0f;
      if (!(dt < 0.0f)) {
        float Tin = 1.0f;
        auto composite = [&](const f32x16& f) {
          const float sigma = fast_softplus(f[0]);
          const float ad = h == 0 ? sigma * dt : 0.0f;
          const float incl = wave_scan_incl(ad, lane);
          const float total = lane_value(incl, 31);
          const float wgt = h == 0 ? Tin * __expf(-(incl - ad)) * (1.0f - __expf(-ad)) : 0.0f;
          cr += wgt * fast_sigmoid(f[1]);
          cg += wgt * fast_sigmoid(f[2]);
          cb += wgt * fast_sigmoid(f[3]);
          Tin = wave_uniform(Tin * __expf(-total));
        };
        // The two chunks of a pair in one pass: chunk b's rows 0..3 move from
        // lanes 0..31 to lanes 32..63 (ds_bpermute: lane l reads lane l % 32),
        // each lane half scans its own 32 samples, and chunk b starts from chunk
        // a's transmittance.  Every sample's weight and colour are computed as by
        // composite(a) then composite(b), in half the instructions; only the
        // final sum over the lanes adds the per-lane colours in another order.
        // The four moves are issued from inline assembly and waited for there:
        // this compiler folded the four ds_bpermute builtins of one MFMA result
        // into one (and its v_permlane32_swap builtin does not model the write
        // to its second register).
        auto composite_pair = [&](const f32x16& fa, const f32x16& fb) {
          float b0, b1, b2, b3;
          const int src = col << 2;
          // fb comes straight from an MFMA: 24 wait states before an LDS
          // instruction reads it (the compiler pads only its own instructions).
          asm volatile(
              "s_nop 7\n"
              "s_nop 7\n"
              "s_nop 7\n"
              "ds_bpermute_b32 %0, %4, %5\n"
              "ds_bpermute_b32 %1, %4, %6\n"
              "ds_bpermute_b32 %2, %4, %7\n"
              "ds_bpermute_b32 %3, %4, %8\n"
              "s_waitcnt lgkmcnt(0)"
              : "=&v"(b0), "=&v"(b1), "=&v"(b2), "=&v"(b3)
              : "v"(src), "v"(fb[0]), "v"(fb[1]), "v"(fb[2]), "v"(fb[3]));
          const float f[4] = {h == 0 ? fa[0] : b0, h == 0 ? fa[1] : b1, h == 0 ? fa[2] : b2, h == 0 ? fa[3] : b3};
          const float sigma = fast_softplus(f[0]);
          const float ad = sigma * dt;
          const float incl = wave_scan_incl32(ad);
          const float total_a = lane_value(incl, 31), total_b = lane_value(incl, 63);
          const float tin_b = wave_uniform(Tin * __expf(-total_a));
          const float wgt = (h == 0 ? Tin : tin_b) * __expf(-(incl - ad)) * (1.0f - __expf(-ad));
          cr += wgt * fast_sigmoid(f[1]);
          cg += wgt * fast_sigmoid(f[2]);
          cb += wgt * fast_sigmoid(f[3]);
          Tin = wave_uniform(tin_b * __expf(-total_b));
        };
        for (int c = 0; c + 1 < chunks; c += 2) {
          const float ta = t0 + (float(32 * c + col) + 0.5f) * dt;
          const float tb = t0 + (float(32 * c + 32 + col) + 0.5f) * dt;
          const float pa[3] = {o[0] + ta * w[0], o[1] + ta * w[1], o[2] + ta * w[2]};
          const float pb[3] = {o[0] + tb * w[0], o[1] + tb * w[1], o[2] + tb * w[2]};
          f32x16 accA[N::kMaxMT], accB[N::kMaxMT];
          half8 bA[N::kMaxKC], bB[N::kMaxKC];
          const LdsWeights ws{sw + opaque_zero(), lane};
          build_input<N>(pa, h, bA);
          if (has_bias) run_pair<N, 0, true, true>(ws, pb, h, bA, bB, accA, accB, sb + opaque_zero());
          else run_pair<N, 0, true, false>(ws, pb, h, bA, bB, accA, accB, sb);
          composite_pair(accA[0], accB[0]);
        }
        if (chunks & 1) {
          const int c = chunks - 1;
          const float ts = t0 + (float(32 * c + col) + 0.5f) * dt;
          const float p[3] = {o[0] + ts * w[0], o[1] + ts * w[1], o[2] + ts * w[2]};
          f32x16 fin[N::kMaxMT];
          eval_chunk<N, true>(sw, sb, has_bias, lane, h, p, fin);
          composite(fin[0]);
        }
        cr = wave_sum(cr);
        cg = wave_sum(cg);
        cb = wave_sum(cb);
      }
      if (lane == 0 && ray < nrays) {
        float* dst = a.image + ray * 3;
        dst[0] = cr;
        dst[1] = cg;
        dst[2] = cb;
      }
    }
    __syncthreads();
  }
}

// --------------------------------------------------------------- compositing
// One wave per ray.  SPL <= 4 samples per lane: lane l owns the SPL consecutive
// samples l SPL .. l SPL + SPL - 1 (one contiguous 16 SPL-byte read, the wave's
// reads one contiguous block), combines them locally and joins the wave scan
// with its partial sum; the next ray's samples are loaded before this ray is
// composited.  Longer rays go through the 64-sample loop.
template <int SPL>
__device__ __forceinline__ void load_ray(const f32x4* __restrict__ src, int samples, int lane, f32x4 (&v)[SPL]) {
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    const int i = lane * SPL + j;
    v[j] = i < samples ? src[i] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }
}

template <int SPL>
__device__ __forceinline__ void composite_ray(const f32x4 (&v)[SPL], float dt, int lane, float* __restrict__ dst) {
  float a[SPL], part = 0.0f;
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    a[j] = v[j][0] * dt;
    part += a[j];
  }
  float run = wave_scan_incl(part, lane) - part;  // optical depth in front of this lane's first sample
  float cr = 0.0f, cg = 0.0f, cb = 0.0f;
#pragma unroll
  for (int j = 0; j < SPL; ++j) {
    const float wgt = __expf(-run) * (1.0f - __expf(-a[j]));
    cr += wgt * v[j][1];
    cg += wgt * v[j][2];
    cb += wgt * v[j][3];
    run += a[j];
  }
  cr = wave_sum(cr);
  cg = wave_sum(cg);
  cb = wave_sum(cb);
  if (lane == 0) {
    dst[0] = cr;
    dst[1] = cg;
    dst[2] = cb;
  }
}

template <int SPL>
__global__ __launch_bounds__(256) void composite_kernel(const f32x4* __restrict__ s, const float* __restrict__ dts,
                                                        int64_t nrays, int samples, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwaves = (int64_t(gridDim.x) * blockDim.x) >> 6;
  if (wave0 >= nrays) return;
  // two register sets, alternating: each ray's samples are requested one ray
  // ahead of its compositing
  f32x4 va[SPL], vb[SPL];
  load_ray<SPL>(s + wave0 * samples, samples, lane, va);
  for (int64_t ray = wave0; ray < nrays; ray += 2 * nwaves) {
    const int64_t rb = ray + nwaves, ra2 = ray + 2 * nwaves;
    if (rb < nrays) load_ray<SPL>(s + rb * samples, samples, lane, vb);
    composite_ray<SPL>(va, dts[ray], lane, out + ray * 3);
    if (ra2 < nrays) load_ray<SPL>(s + ra2 * samples, samples, lane, va);
    if (rb < nrays) composite_ray<SPL>(vb, dts[rb], lane, out + rb * 3);
  }
}

#if RDV_FIELD_PART == 0
__global__ __launch_bounds__(256) void composite_long_kernel(const f32x4* __restrict__ s,
                                                             const float* __restrict__ dts, int64_t nrays,
                                                             int samples, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;
  const int64_t nwaves = (int64_t(gridDim.x) * blockDim.x) >> 6;
  for (int64_t ray = wave0; ray < nrays; ray += nwaves) {
    const float dt = dts[ray];
    const f32x4* src = s + ray * samples;
    float Tin = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
    for (int k = 0; k < samples; k += 64) {
      const int i = k + lane;
      f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
      if (i < samples) v = src[i];
      const float ad = v[0] * dt;
      const float incl = wave_scan_incl(ad, lane);
      const float total = lane_value(incl, 63);
      const float wgt = Tin * __expf(-(incl - ad)) * (1.0f - __expf(-ad));
      cr += wgt * v[1];
      cg += wgt * v[2];
      cb += wgt * v[3];
      Tin *= __expf(-total);
    }
    cr = wave_sum(cr);
    cg = wave_sum(cg);
    cb = wave_sum(cb);
    if (lane == 0) {
      out[ray * 3 + 0] = cr;
      out[ray * 3 + 1] = cg;
      out[ray * 3 + 2] = cb;
    }
  }
}
#endif

// ------------------------------------------------ raymarching transmittance
struct TransmittanceArgs {
  const float* rays;  // [n, 6]: x, w (world)
  int64_t nrays;
  const uint8_t* packed;
  MlpLayout lay;
  float M[12];        // mat4x3, column-major: linear columns 0..2, translation column 3
  float step, density_scale;
  float* out;         // [n]
  int lane_rays;      // 1: one ray per MFMA column (raymarch_rays_lanes), 0: one ray per wave
};

// The reference marches sequentially (transmittance_rm):
//   for (k = 0; d > 0 && k < 4096; k++) { tau += extinction(x) * density * step;
//     if (tau > 16) return 0; d -= step; x += step * w; }   return exp(-tau)
// with every update rounded to fp32.  Here a chunk of 32 consecutive steps is
// one MFMA block: lane c reproduces x_{k0+c} and d_{k0+c} by applying the same
// fp32 updates c times (so the sample positions and the step count are the
// reference's, bit for bit), the 32 extinctions are evaluated together, and tau
// is an inclusive wavefront scan of the increments (the order of that fp32 sum
// is the only difference from the reference).
// The march of every ray of this block: sigma_of(x) returns this lane's
// extinction at its sample position x (lanes l and l + 32 hold the same sample;
// the value of lanes 0..31 is used).
template <class Sigma>
__device__ __forceinline__ void raymarch_rays_chunks(const TransmittanceArgs& a, int* s_next, Sigma&& sigma_of) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  const BlockRays br(a.nrays);
  const int nr = br.count;
  float L[9];
  inverse3(a.M, L);
  auto claim = [&]() {
    int t = 0;
    if (lane == 0) t = atomicAdd(s_next, 1);
    return __builtin_amdgcn_readfirstlane(t);
  };
  for (int r = claim(); r < nr; r = claim()) {
    const int64_t ray = br.ray(r);
    if (ray >= a.nrays) continue;
    const float* rr = a.rays + ray * 6;
    const float xw[3] = {rr[0] - a.M[9], rr[1] - a.M[10], rr[2] - a.M[11]};
    float x[3], w[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {  // L * v with L column-major
      x[i] = L[i] * xw[0] + L[3 + i] * xw[1] + L[6 + i] * xw[2];
      w[i] = L[i] * rr[3] + L[3 + i] * rr[4] + L[6 + i] * rr[5];
    }
    float tmin, tmax;
    ray_box(x, w, tmin, tmax);
    float T = 1.0f;
    if (!(tmax <= 0.0f || tmin > tmax)) {
      tmin = fmaxf(0.0f, tmin);
      float sws[3];
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        float wt = w[i] * tmin;
        asm volatile("" : "+v"(wt));  // x += w * tMin: product and sum rounded separately
        x[i] = x[i] + wt;
        sws[i] = a.step * w[i];
        asm volatile("" : "+v"(sws[i]));  // the product is rounded on its own, as x += step * w
      }
      float d = tmax - tmin;
      float tau = 0.0f;
      bool dead = false;
      for (int k0 = 0; k0 < 4096 && d > 0.0f; k0 += 32) {
        // lane c: position and remaining distance after c more steps
        float xc[3] = {x[0], x[1], x[2]}, dc = d;
        for (int it = 0; it < 31; ++it) {
          if (it < col) {
            dc = dc - a.step;
#pragma unroll
            for (int i = 0; i < 3; ++i) xc[i] = xc[i] + sws[i];
          }
        }
        const bool valid = dc > 0.0f && k0 + col < 4096;
        // every lane in [0, c) was valid when lane c is (d only decreases)
        const float sigma = sigma_of(xc);
        const float ce = sigma * a.density_scale;
        float inc = ce * a.step;
        asm volatile("" : "+v"(inc));
        inc = (h == 0 && valid) ? inc : 0.0f;
        const float incl = tau + wave_scan_incl(inc, lane);
        const bool over = h == 0 && valid && incl > 16.0f;
        if (__builtin_amdgcn_ballot_w64(over) != 0) {
          dead = true;
          break;
        }
        const uint64_t vmask = __builtin_amdgcn_ballot_w64(h == 0 && valid);
        const int last = 63 - __builtin_clzll(vmask);  // highest valid lane (lane 0 is valid here)
        tau = lane_value(incl, last);
        if (last < 31) break;  // the march ended inside this chunk
        // state after step k0 + 31, then one more step: the next chunk's start
        float nd = lane_value(dc, 31);
        float nx[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) nx[i] = lane_value(xc[i], 31);
        d = nd - a.step;
#pragma unroll
        for (int i = 0; i < 3; ++i) x[i] = nx[i] + sws[i];
      }
      T = dead ? 0.0f : expf(-tau);
    }
    if (lane == 0) a.out[ray] = T;
  }
}

// One ray of a lane-per-ray march (lanes l and l + 32 hold the same ray).
struct MarchRay {
  float x[3], sw[3];  // object-space position, step * w
  float d, tau;       // distance left, optical depth
  int k;              // steps taken
};

// The start of ray `ray`: the same fp32 operations as raymarch_rays_chunks
// (false: the ray misses the box, T = 1).
__device__ __forceinline__ bool march_start(const TransmittanceArgs& a, const float (&L)[9], int64_t ray,
                                            MarchRay& r) {
  const float* rr = a.rays + ray * 6;
  const float xw[3] = {rr[0] - a.M[9], rr[1] - a.M[10], rr[2] - a.M[11]};
  float w[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {  // L * v with L column-major
    r.x[i] = L[i] * xw[0] + L[3 + i] * xw[1] + L[6 + i] * xw[2];
    w[i] = L[i] * rr[3] + L[3 + i] * rr[4] + L[6 + i] * rr[5];
  }
  float tmin, tmax;
  ray_box(r.x, w, tmin, tmax);
  if (tmax <= 0.0f || tmin > tmax) return false;
  tmin = fmaxf(0.0f, tmin);
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    float wt = w[i] * tmin;
    asm volatile("" : "+v"(wt));  // x += w * tMin: product and sum rounded separately
    r.x[i] = r.x[i] + wt;
    r.sw[i] = a.step * w[i];
    asm volatile("" : "+v"(r.sw[i]));  // the product is rounded on its own, as x += step * w
  }
  r.d = tmax - tmin;
  r.tau = 0.0f;
  r.k = 0;
  return true;
}

// The same march with one ray per MFMA column: each lane takes one step of its
// own ray per evaluation of the extinction chain, in the reference's order
// (tau summed sequentially, so T is the reference's fp32 result up to the
// extinction values).  A column whose ray ends claims the next ray of the
// block's range at once.  No replay of the position updates: for launches with
// several rays per column (the host picks this mode from the ray count); with
// few rays per column a ray's steps would each wait for a whole chain, where
// raymarch_rays_chunks takes 32 of them per chain.
template <class Sigma>
__device__ __forceinline__ void raymarch_rays_lanes(const TransmittanceArgs& a, int* s_next, Sigma&& sigma_of) {
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  const BlockRays br(a.nrays);
  const int nr = br.count;
  float L[9];
  inverse3(a.M, L);
  MarchRay r;
#pragma unroll
  for (int i = 0; i < 3; ++i) r.x[i] = r.sw[i] = 0.0f;
  r.d = r.tau = 0.0f;
  r.k = 0;
  int64_t ray = -1;        // the ray in this column (-1: none)
  bool exhausted = false;  // the block's range has run dry
  const uint64_t below = (uint64_t(1) << col) - 1;
  auto finish = [&](float T) {
    if (h == 0) a.out[ray] = T;
    ray = -1;
  };
  for (;;) {
    // Fill: columns without a ray take the next ones of the range.
    for (;;) {
      const bool idle = ray < 0 && !exhausted;
      const uint64_t want = __builtin_amdgcn_ballot_w64(h == 0 && idle);
      if (want == 0) break;
      int base = 0;
      if (lane == 0) base = atomicAdd(s_next, __builtin_popcountll(want));
      base = __builtin_amdgcn_readfirstlane(base);
      if (idle) {  // both halves see the same `want` bits of the h == 0 lanes
        const int k = base + __builtin_popcountll(want & below);
        if (k < nr) {
          ray = br.ray(k);
          if (ray >= a.nrays) ray = -1;  // past the last ray: claim again
          else if (!march_start(a, L, ray, r) || !(r.d > 0.0f)) finish(1.0f);  // no step: exp(-0)
        } else {
          exhausted = true;
        }
      }
    }
    if (__builtin_amdgcn_ballot_w64(h == 0 && ray >= 0) == 0) break;  // every column is out of work
    float p[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) p[i] = ray >= 0 ? r.x[i] : 0.0f;
    float sigma = sigma_of(p);
    sigma = __shfl(sigma, col);  // the value of lane col (row 0 of its column)
    if (ray >= 0) {
      const float ce = sigma * a.density_scale;
      float inc = ce * a.step;
      asm volatile("" : "+v"(inc));
      r.tau = r.tau + inc;
      if (r.tau > 16.0f) {
        finish(0.0f);
      } else {
        r.d = r.d - a.step;
#pragma unroll
        for (int i = 0; i < 3; ++i) r.x[i] = r.x[i] + r.sw[i];
        ++r.k;
        if (!(r.d > 0.0f && r.k < 4096)) finish(expf(-r.tau));
      }
    }
  }
}

template <class Sigma>
__device__ __forceinline__ void raymarch_rays(const TransmittanceArgs& a, int* s_next, Sigma&& sigma_of) {
  if (a.lane_rays) raymarch_rays_lanes(a, s_next, sigma_of);
  else raymarch_rays_chunks(a, s_next, sigma_of);
}

template <class N, int HEAD_ACT>
__global__ __launch_bounds__(kRenderThreads, 1) void raymarch_transmittance_kernel(TransmittanceArgs a) {
  static_assert(N::kIn == 3 && N::kOut == 1, "the extinction is a Map[3, 1]");
  __shared__ float sb[N::kBias];
  __shared__ half8 sw[N::kFrags * 64];
  __shared__ int s_next;
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5;
  const bool has_bias = packed_has_bias(a.packed);
  stage_weights<N, kRenderThreads>(a.packed, a.lay, sb, sw, &s_next);
  raymarch_rays(a, &s_next, [&](const float (&xc)[3]) {
    f32x16 fin[N::kMaxMT];
    eval_chunk<N, true>(sw, sb, has_bias, lane, h, xc, fin);
    return head_act<HEAD_ACT>(0, fin[0][0]);
  });
}

// ------------------------------------------- runtime-shaped fields (mlp_generic.h)
// Any LinearFast field or extinction chain without a compile-time instance:
// the same per-ray work, with each 32-sample chunk evaluated by gen_chain.
struct TransmittanceGenArgs {
  TransmittanceArgs t;
  GenNet net;
};

template <int MT, bool LDSW, bool F32L = false>
__global__ __launch_bounds__(64 * gen_waves<MT>(), 1) void raymarch_generic_kernel(TransmittanceGenArgs ga) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_next;
  const TransmittanceArgs& a = ga.t;
  const GenNet& g = ga.net;
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5;
  const bool has_bias = packed_has_bias(a.packed);
  const half8* w0;
  const float* b0;
  gen_sources<LDSW>(a.packed, g, smem, &w0, &b0);
  if (threadIdx.x == 0) s_next = 0;
  __syncthreads();
  const int act = g.act[g.L - 1];
  raymarch_rays(a, &s_next, [&](const float (&xc)[3]) {
    return gen_field_row0<MT, F32L>(g, w0, b0, has_bias, lane, h, xc, act);
  });
}

// ------------------------------------------------ ratio-tracking transmittance
// RatiotrackingTransmittance with a VoxelMajorantField (src/rdv/domain/volumes.py:144-211,
// shaders/volumes/ratiotracking_transmittance.h, ratiotracking_transmittance_trait.h,
// voxel_majorant_field.h).  Per ray, in the object space of the transform,
// from the box entry with d = tMax - max(0, tMin) left to travel:
//   for (safety = 0; d > 0 && safety < 1024; safety++) {
//     (maj, dist) = majorant(x, w);  maj = max(maj, 1e-12);  dist = max(dist, 1e-6)
//     dt = min(dist, -log(1 - random()) / (maj * density_scale));  d -= dt;  x += dt * w
//     if (dt >= dist) continue;            // left the majorant voxel first
//     if (d <= 0) break;                   // left the box first
//     T *= 1 - extinction(x) / maj
//     if (T < 0.05) { if (random() >= T) return 0;  T = 1; }   // Russian roulette
//   }
//   return T
// Every update is rounded to fp32 on its own (no contraction), so sample
// positions, voxel choices and random draws follow the reference's arithmetic.
//
// Mapping: a wave tracks 32 rays at once, one per MFMA column (lanes l and
// l + 32 mirror ray l).  Each lane runs its ray's free flights on its own until
// it needs an extinction value; then the wave evaluates the extinction chain
// once for all 32 pending positions on the matrix cores.  A lane whose ray ends
// claims the next ray of the block's range at once, so the 32 columns stay
// filled until the range runs dry.
struct RatioArgs {
  const float* rays;      // [n, 6]: x, w (world)
  int64_t nrays;
  const float* majorant;  // [D, H, W] fp32: one upper bound of the extinction per voxel of [-1,1]^3
  int mw, mh, md;         // W, H, D
  float M[12];            // mat4x3, column-major
  float density_scale;
  uint32_t seeds[4];      // the dispatch's random seeds
  int rng_skip;           // random() draws a thread has taken before this map (2 after a jittered camera)
  float* out;             // [n]
};

// One ray of a ratio-tracking wave: its free flights run per lane.
struct RatioRay {
  float x[3], w[3];
  float d, T, maj;
  int safety;
  RngState st;
};

// Free flights until the next collision (true: x is the collision point and
// `maj` its majorant) or the end of the ray (false: T is the result).
__device__ __forceinline__ bool ratio_flight(const RatioArgs& a, RatioRay& r) {
#pragma clang fp contract(off)
  for (;;) {
    if (!(r.d > 0.0f && r.safety < 1024)) return false;
    float dist;
    float mj = voxel_majorant(a.majorant, a.mw, a.mh, a.md, r.x, r.w, dist);
    mj = fmaxf(mj, 1e-12f);
    dist = fmaxf(dist, 1e-6f);
    const float u = rng_uniform(r.st);
    const float ff = -logf(1.0f - u) / (mj * a.density_scale);
    const float dt = fminf(dist, ff);
    r.d = r.d - dt;
#pragma unroll
    for (int i = 0; i < 3; ++i) r.x[i] = r.x[i] + dt * r.w[i];
    ++r.safety;
    if (dt >= dist) continue;
    if (r.d <= 0.0f) return false;
    r.maj = mj;
    return true;
  }
}

// The start of ray `ray`: object-space entry point (false: the ray misses, T = 1).
__device__ __forceinline__ bool ratio_start(const RatioArgs& a, const float (&L)[9], int64_t ray, RatioRay& r) {
  const float* rr = a.rays + ray * 6;
  const float xw[3] = {rr[0] - a.M[9], rr[1] - a.M[10], rr[2] - a.M[11]};
#pragma unroll
  for (int i = 0; i < 3; ++i) {  // L * v with L column-major
    r.x[i] = L[i] * xw[0] + L[3 + i] * xw[1] + L[6 + i] * xw[2];
    r.w[i] = L[i] * rr[3] + L[3 + i] * rr[4] + L[6 + i] * rr[5];
  }
  r.T = 1.0f;
  r.safety = 0;
  r.st = rng_spawn(a.seeds, int(ray));
  for (int k = 0; k < a.rng_skip; ++k) rng_step(r.st);
  float tmin, tmax;
  ray_box(r.x, r.w, tmin, tmax);
  if (tmax <= 0.0f || tmin > tmax) return false;
  tmin = fmaxf(0.0f, tmin);
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    float wt = r.w[i] * tmin;
    asm volatile("" : "+v"(wt));  // x += w * tMin: product and sum rounded separately
    r.x[i] = r.x[i] + wt;
  }
  r.d = tmax - tmin;
  return true;
}

struct RatioGenArgs {
  RatioArgs r;
  const uint8_t* packed;
  GenNet net;
};

template <int MT, bool LDSW, bool F32L = false>
__global__ __launch_bounds__(64 * gen_waves<MT>(), 1) void ratiotracking_generic_kernel(RatioGenArgs ga) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_next;
  const RatioArgs& a = ga.r;
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

  RatioRay r;
#pragma unroll
  for (int i = 0; i < 3; ++i) r.x[i] = r.w[i] = 0.0f;
  r.d = r.T = r.maj = 0.0f;
  r.safety = 0;
  r.st = RngState{0, 0, 0, 0};
  int64_t ray = -1;        // the ray in this column (-1: none)
  bool pending = false;    // x is a collision point waiting for its extinction
  bool exhausted = false;  // the block's range has run dry
  const uint64_t below = (uint64_t(1) << col) - 1;
  auto finish = [&](float T) {
    if (h == 0) a.out[ray] = T;
    ray = -1;
  };
  for (;;) {
    // Fill: advance every ray to its next collision; columns that run out of
    // ray take the next ones of the range.
    for (;;) {
      if (ray >= 0 && !pending) {
        if (ratio_flight(a, r)) pending = true;
        else finish(r.T);
      }
      const bool idle = ray < 0 && !exhausted;
      const uint64_t want = __builtin_amdgcn_ballot_w64(h == 0 && idle);
      if (want == 0) break;
      int base = 0;
      if (lane == 0) base = atomicAdd(&s_next, __builtin_popcountll(want));
      base = __builtin_amdgcn_readfirstlane(base);
      if (idle) {  // both halves see the same `want` bits of the h == 0 lanes
        const int k = base + __builtin_popcountll(want & below);
        if (k < nr) {
          ray = br.ray(k);
          if (ray >= a.nrays) ray = -1;  // past the last ray: claim again
          else if (!ratio_start(a, L, ray, r)) finish(1.0f);
        } else {
          exhausted = true;
        }
      }
    }
    if (__builtin_amdgcn_ballot_w64(h == 0 && pending) == 0) break;  // every column is out of work
    float p[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) p[i] = pending ? r.x[i] : 0.0f;
    float sigma = gen_field_row0<MT, F32L>(g, w0, b0, has_bias, lane, h, p, act);
    sigma = __shfl(sigma, col);  // the value of lane col (row 0 of its column)
    if (pending) {
#pragma clang fp contract(off)
      pending = false;
      r.T = r.T * (1.0f - sigma / r.maj);
      if (r.T < 0.05f) {
        if (rng_uniform(r.st) >= r.T) finish(0.0f);
        else r.T = 1.0f;
      }
    }
  }
}

struct RenderGenArgs {
  RenderArgs r;
  GenNet net;
};

// Emission-absorption render with a runtime-shaped field (raw 4-wide head):
// one ray per wave at a time, one 32-sample chunk per chain evaluation.
template <int MT, bool LDSW>
__global__ __launch_bounds__(64 * gen_waves<MT>(), 1) void render_ea_generic_kernel(RenderGenArgs ga) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_next;
  const RenderArgs& a = ga.r;
  const GenNet& g = ga.net;
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  const int64_t nrays = ea_ray_count(a);
  const BlockRays br(nrays, false);
  const int nr = br.count;
  const bool has_bias = packed_has_bias(a.packed);
  const half8* w0;
  const float* b0;
  gen_sources<LDSW>(a.packed, g, smem, &w0, &b0);
  if (threadIdx.x == 0) s_next = 0;
  __syncthreads();
  auto claim = [&]() {
    int t = 0;
    if (lane == 0) t = atomicAdd(&s_next, 1);
    return __builtin_amdgcn_readfirstlane(t);
  };
  const int chunks = a.samples / 32;
  for (int r = claim(); r < nr; r = claim()) {
    const int64_t ray = br.ray(r);
    if (ray >= nrays) continue;
    float o[3], w[3];
    ea_ray(a, ray, o, w);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      o[i] = wave_uniform(o[i]);
      w[i] = wave_uniform(w[i]);
    }
    float t0, t1;
    ray_box(o, w, t0, t1);
    float cr = 0.0f, cg = 0.0f, cb = 0.0f;
    if (!(t1 <= 0.0f || t0 > t1)) {
      t0 = wave_uniform(fmaxf(t0, 0.0f));
      const float dt = wave_uniform((t1 - t0) / float(a.samples));
      float Tin = 1.0f;
      for (int c = 0; c < chunks; ++c) {
        const float ts = t0 + (float(32 * c + col) + 0.5f) * dt;
        const float p[3] = {o[0] + ts * w[0], o[1] + ts * w[1], o[2] + ts * w[2]};
        const int z = opaque_zero();
        const half8* wsrc = w0 + z;
        auto wf = [&](int f) { return wsrc[f * 64 + lane]; };
        auto get = [&](int d) { return d == 0 ? p[0] : (d == 1 ? p[1] : p[2]); };
        auto l0 = [&](int cc) { return gen_l0_chunk(g, cc, h, get); };
        f32x4 o4 = {0.0f, 0.0f, 0.0f, 0.0f};
        auto sink = [&](const auto& acc) {
#pragma unroll
          for (int j = 0; j < 4; ++j) o4[j] = acc[0][j];
        };
        gen_chain<MT>(g, GenCtx{b0 + z, has_bias, h}, wf, l0, sink);
        // rows 0..3 (density, RGB logits) sit in registers 0..3 of lanes 0..31
        const float sigma = fast_softplus(o4[0]);
        const float ad = h == 0 ? sigma * dt : 0.0f;
        const float incl = wave_scan_incl(ad, lane);
        const float total = lane_value(incl, 31);
        const float wgt = h == 0 ? Tin * __expf(-(incl - ad)) * (1.0f - __expf(-ad)) : 0.0f;
        cr += wgt * fast_sigmoid(o4[1]);
        cg += wgt * fast_sigmoid(o4[2]);
        cb += wgt * fast_sigmoid(o4[3]);
        Tin *= __expf(-total);
      }
      cr = wave_sum(cr);
      cg = wave_sum(cg);
      cb = wave_sum(cb);
    }
    if (lane == 0) {
      float* dst = a.image + ray * 3;
      dst[0] = cr;
      dst[1] = cg;
      dst[2] = cb;
    }
  }
}

// ---------------------------------------------------------- instantiations
// 8-tile launchers of the runtime-shaped field kernels (RDV_FIELD_PART 1..3).
int launch_raymarch_generic8(const TransmittanceGenArgs& a, int64_t items, int cu, int64_t lds, bool in_lds,
                             hipStream_t stream);
int launch_ratiotracking_generic8(const RatioGenArgs& a, int64_t items, int cu, int64_t lds, bool in_lds,
                                  hipStream_t stream);
int launch_render_ea_generic8(const RenderGenArgs& a, int64_t items, int cu, int64_t lds, bool in_lds,
                              hipStream_t stream);

#if RDV_FIELD_PART == 0
using RenderNet64x3 = Net<RDV_ENC_NONE, 3, 0, 4, 1, 2, 2, 2, 1>;   // 3->64->64->64->4
using ExtinctionNet64x3 = Net<RDV_ENC_NONE, 3, 0, 1, 1, 2, 2, 2, 1>;  // 3->64->64->64->1

// Is `d` the renderer's field network: 3 -> 64 -> 64 -> 64 -> 4, fp16, ReLU
// hidden activations, raw (no-activation) head (softplus / sigmoid are applied
// by the renderer)?
static bool is_render_field(const rdv_mlp_desc& d, const MlpLayout& lay) {
  if (d.encoding != RDV_ENC_NONE || d.in_features != 3 || d.n_layers != 4) return false;
  const int dims[5] = {3, 64, 64, 64, 4};
  for (int i = 0; i <= 4; ++i)
    if (d.dims[i] != dims[i]) return false;
  for (int i = 0; i < 4; ++i)
    if (d.prec[i] != RDV_PREC_F16) return false;
  for (int i = 0; i < 3; ++i)
    if (d.act[i] != RDV_ACT_RELU) return false;
  return d.act[3] == RDV_ACT_NONE && lay.kc[0] == 1;
}

static bool is_extinction_field(const rdv_mlp_desc& d, const MlpLayout& lay) {
  if (d.encoding != RDV_ENC_NONE || d.in_features != 3 || d.n_layers != 4) return false;
  const int dims[5] = {3, 64, 64, 64, 1};
  for (int i = 0; i <= 4; ++i)
    if (d.dims[i] != dims[i]) return false;
  for (int i = 0; i < 4; ++i)
    if (d.prec[i] != RDV_PREC_F16) return false;
  for (int i = 0; i < 3; ++i)
    if (d.act[i] != RDV_ACT_RELU) return false;
  return (d.act[3] == RDV_ACT_NONE || d.act[3] == RDV_ACT_SOFTPLUS || d.act[3] == RDV_ACT_RELU) && lay.kc[0] == 1;
}

__global__ void random_uniform_kernel(JitterSeeds js, int64_t n_threads, int per_thread, float* __restrict__ out) {
  for (int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; t < n_threads; t += int64_t(gridDim.x) * blockDim.x) {
    RngState st = rng_spawn(js.seeds, int(t));
    for (int k = 0; k < per_thread; ++k) out[t * per_thread + k] = rng_uniform(st);
  }
}

int launch_random_uniform(const uint32_t* seeds, int64_t n_threads, int per_thread, float* out, hipStream_t stream) {
  JitterSeeds js{1, {seeds[0], seeds[1], seeds[2], seeds[3]}};
  int64_t blocks = (n_threads + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  random_uniform_kernel<<<dim3(unsigned(blocks)), dim3(256), 0, stream>>>(js, n_threads, per_thread, out);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

int launch_camera_rays(const rdv_camera_desc& c, const float* poses, const uint32_t* seeds, float* rays,
                       hipStream_t stream) {
  CameraParams p{poses, c.n_cams, c.height, c.width, c.aspect_ratio, c.fov};
  JitterSeeds js{0, {0, 0, 0, 0}};
  if (seeds != nullptr) js = JitterSeeds{1, {seeds[0], seeds[1], seeds[2], seeds[3]}};
  const int64_t total = int64_t(c.n_cams) * c.height * c.width;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  camera_rays_kernel<<<dim3(unsigned(blocks)), dim3(256), 0, stream>>>(p, js, rays);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

int launch_render_ea(const rdv_camera_desc& c, const float* poses, const float* rays, int64_t n_rays,
                     const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, int samples, float* image,
                     hipStream_t stream) {
  const bool fixed = is_render_field(d, lay);
  if (!fixed && !(is_f16_field(d, 4) && d.act[d.n_layers - 1] == RDV_ACT_NONE))
    return fail(RDV_ERR_UNSUPPORTED,
                "the renderer's field must be a LinearFast chain from 3 inputs to 4 raw outputs (density and RGB "
                "logits; the renderer applies softplus and sigmoid)");
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  RenderArgs a;
  a.cam = CameraParams{poses, c.n_cams, c.height, c.width, c.aspect_ratio, c.fov};
  a.rays = rays;
  a.n_rays = n_rays;
  a.packed = static_cast<const uint8_t*>(packed);
  a.lay = lay;
  a.image = image;
  a.samples = samples;
  const int64_t nrays = rays != nullptr ? n_rays : int64_t(c.n_cams) * c.height * c.width;
  if (!fixed) {
    RenderGenArgs ga;
    ga.r = a;
    gen_net(d, lay, &ga.net);
    RDV_GEN_FIELD_DISPATCH(render_ea_generic_kernel, ga, nrays, di.cu_count, ga.net, stream,
                           launch_render_ea_generic8);
  }
  int64_t blocks = di.cu_count;
  const int64_t need = (nrays + kEaWaves - 1) / kEaWaves;
  if (need < blocks) blocks = need;
  render_ea_kernel<RenderNet64x3><<<dim3(unsigned(blocks)), dim3(kEaThreads), 0, stream>>>(a);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

int launch_composite(const float* sigma_rgb, const float* dts, int64_t nrays, int samples, float* out,
                     hipStream_t stream) {
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  int64_t blocks = (nrays + 3) / 4;  // 4 waves (rays) per block
  const int64_t cap = int64_t(di.cu_count) * 8;
  if (blocks > cap) blocks = cap;
  const dim3 grid(static_cast<unsigned>(blocks)), block(256);
  const f32x4* s = reinterpret_cast<const f32x4*>(sigma_rgb);
  if (samples <= 64) composite_kernel<1><<<grid, block, 0, stream>>>(s, dts, nrays, samples, out);
  else if (samples <= 128) composite_kernel<2><<<grid, block, 0, stream>>>(s, dts, nrays, samples, out);
  else if (samples <= 256) composite_kernel<4><<<grid, block, 0, stream>>>(s, dts, nrays, samples, out);
  else composite_long_kernel<<<grid, block, 0, stream>>>(s, dts, nrays, samples, out);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

int launch_raymarch_transmittance(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, const float* rays,
                                  int64_t nrays, const float* transform12, float step, float density_scale,
                                  float* out, hipStream_t stream) {
  const bool fixed = is_extinction_field(d, lay);
  std::string why;
  const bool mixed = !fixed && is_mixed_field(d, lay, 1, &why);
  if (!fixed && !mixed && !is_f16_field(d, 1))
    return fail(RDV_ERR_UNSUPPORTED, why.empty() ? "the extinction must be a chain of LinearFast / Linear layers from 3 "
                                                   "inputs to 1 output" : why);
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  TransmittanceArgs a;
  a.rays = rays;
  a.nrays = nrays;
  a.packed = static_cast<const uint8_t*>(packed);
  a.lay = lay;
  for (int i = 0; i < 12; ++i) a.M[i] = transform12[i];
  a.step = step;
  a.density_scale = density_scale;
  a.out = out;
  // One ray per MFMA column once every column of a full grid gets two rays or
  // more (8 waves per block for the runtime-shaped kernels, at most).
  a.lane_rays = nrays >= int64_t(2) * 32 * (fixed ? kRenderWaves : 8) * di.cu_count ? 1 : 0;
  if (!fixed) {
    TransmittanceGenArgs ga;
    ga.t = a;
    gen_net(d, lay, &ga.net);
    if (mixed) RDV_GEN_FIELD_DISPATCH_MIXED(raymarch_generic_kernel, ga, nrays, di.cu_count, ga.net, stream);
    RDV_GEN_FIELD_DISPATCH(raymarch_generic_kernel, ga, nrays, di.cu_count, ga.net, stream,
                           launch_raymarch_generic8);
  }
  int64_t blocks = di.cu_count;
  const int64_t need = (nrays + kRenderWaves - 1) / kRenderWaves;
  if (need < blocks) blocks = need;
  const dim3 grid(static_cast<unsigned>(blocks)), block(static_cast<unsigned>(kRenderThreads));
  switch (d.act[3]) {
    case RDV_ACT_SOFTPLUS:
      raymarch_transmittance_kernel<ExtinctionNet64x3, RDV_ACT_SOFTPLUS><<<grid, block, 0, stream>>>(a);
      break;
    case RDV_ACT_RELU:
      raymarch_transmittance_kernel<ExtinctionNet64x3, RDV_ACT_RELU><<<grid, block, 0, stream>>>(a);
      break;
    default:
      raymarch_transmittance_kernel<ExtinctionNet64x3, RDV_ACT_NONE><<<grid, block, 0, stream>>>(a);
      break;
  }
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}


__global__ __launch_bounds__(256) void voxel_majorant_kernel(const float* __restrict__ grid, int mw, int mh, int md,
                                                             const float* __restrict__ rays, int64_t n,
                                                             float* __restrict__ out) {
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    const float* rr = rays + i * 6;
    const float x[3] = {rr[0], rr[1], rr[2]}, w[3] = {rr[3], rr[4], rr[5]};
    float dist;
    const float m = voxel_majorant(grid, mw, mh, md, x, w, dist);
    out[2 * i] = m;
    out[2 * i + 1] = dist;
  }
}

int launch_voxel_majorant(const float* grid, int mw, int mh, int md, const float* rays, int64_t n, float* out,
                          hipStream_t stream) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  voxel_majorant_kernel<<<dim3(unsigned(blocks)), dim3(256), 0, stream>>>(grid, mw, mh, md, rays, n, out);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

int launch_ratiotracking(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed,
                         const rdv_ratiotracking_desc& rt, const float* majorant, const float* rays, int64_t nrays,
                         float* out, hipStream_t stream) {
  std::string why;
  const bool mixed = is_mixed_field(d, lay, 1, &why);
  if (!mixed && !is_f16_field(d, 1))
    return fail(RDV_ERR_UNSUPPORTED, why.empty() ? "the extinction must be a chain of LinearFast / Linear layers from 3 "
                                                   "inputs to 1 output" : why);
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  RatioGenArgs ga;
  RatioArgs& a = ga.r;
  a.rays = rays;
  a.nrays = nrays;
  a.majorant = majorant;
  a.mw = rt.maj_width;
  a.mh = rt.maj_height;
  a.md = rt.maj_depth;
  for (int i = 0; i < 12; ++i) a.M[i] = rt.transform[i];
  a.density_scale = rt.density_scale;
  for (int i = 0; i < 4; ++i) a.seeds[i] = rt.seeds[i];
  a.rng_skip = rt.rng_skip;
  a.out = out;
  ga.packed = static_cast<const uint8_t*>(packed);
  gen_net(d, lay, &ga.net);
  // 32 rays per wave
  if (mixed) RDV_GEN_FIELD_DISPATCH_MIXED(ratiotracking_generic_kernel, ga, (nrays + 31) / 32, di.cu_count, ga.net, stream);
  RDV_GEN_FIELD_DISPATCH(ratiotracking_generic_kernel, ga, (nrays + 31) / 32, di.cu_count, ga.net, stream,
                         launch_ratiotracking_generic8);
}

// ------------------------------------------------------------- majorant grid
struct MajorantGridArgs {
  const float* fine;
  float* out;
  int rank, channels, aligned, linear;
  int fshape[4], cshape[4];
  int64_t cells;
};

// majorant_grid.h: the fine index range [lo, lo + ext) along one dimension that
// a sampler can read from inside coarse cell i of n.
__device__ __forceinline__ void majorant_range(int i, int n, int fine, bool aligned, bool lin, int& lo, int& ext) {
#pragma clang fp contract(off)
  const float fsz = float(fine);
  const float t_lo = float(i) / float(n);
  const float t_hi = float(i + 1) / float(n);
  const float pos_lo = aligned ? t_lo * (fsz - 1.0f) : t_lo * fsz - 0.5f;
  const float pos_hi = aligned ? t_hi * (fsz - 1.0f) : t_hi * fsz - 0.5f;
  int d_lo, d_hi;
  if (lin) {
    d_lo = int(floorf(pos_lo));
    d_hi = int(floorf(pos_hi)) + 2;
  } else {
    d_lo = int(floorf(pos_lo + 0.5f));
    d_hi = int(floorf(pos_hi + 0.5f)) + 1;
  }
  if (d_lo < 0) d_lo = 0;
  if (d_hi > fine) d_hi = fine;
  if (d_hi <= d_lo) d_hi = d_lo + 1;
  if (d_hi > fine) d_hi = fine;
  if (d_lo >= d_hi) d_lo = d_hi - 1;
  lo = d_lo;
  ext = d_hi - d_lo;
}

// One wave per coarse cell: the lanes stride over the cell's fine window and
// the maxima meet in a butterfly (max is exact, so the order does not matter).
__global__ __launch_bounds__(256) void majorant_grid_kernel(MajorantGridArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t waves = int64_t(gridDim.x) * (blockDim.x >> 6);
  for (int64_t c = int64_t(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6); c < a.cells; c += waves) {
    int lo[4] = {0, 0, 0, 0}, ext[4] = {1, 1, 1, 1};
    int64_t rem = c, count = 1;
    for (int d = a.rank - 1; d >= 0; --d) {
      const int idx = int(rem % a.cshape[d]);
      rem /= a.cshape[d];
      majorant_range(idx, a.cshape[d], a.fshape[d], a.aligned != 0, a.linear != 0, lo[d], ext[d]);
      count *= ext[d];
    }
    for (int k = 0; k < a.channels; ++k) {
      float m = -INFINITY;
      for (int64_t j = lane; j < count; j += 64) {
        int64_t r = j, flat = 0, stride = 1;
        for (int d = a.rank - 1; d >= 0; --d) {
          const int64_t id = lo[d] + r % ext[d];
          r /= ext[d];
          flat += id * stride;
          stride *= a.fshape[d];
        }
        m = fmaxf(m, a.fine[flat * a.channels + k]);
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
      if (lane == 0) a.out[c * a.channels + k] = m;
    }
  }
}

int launch_majorant_grid(const rdv_majorant_grid_desc& g, const float* fine, float* out, hipStream_t stream) {
  MajorantGridArgs a;
  a.fine = fine;
  a.out = out;
  a.rank = g.rank;
  a.channels = g.channels;
  a.aligned = g.aligned;
  a.linear = g.linear;
  a.cells = 1;
  for (int d = 0; d < 4; ++d) {
    a.fshape[d] = d < g.rank ? g.fine_shape[d] : 1;
    a.cshape[d] = d < g.rank ? g.shape[d] : 1;
    if (d < g.rank) a.cells *= g.shape[d];
  }
  if (a.cells == 0) return RDV_OK;
  int64_t blocks = (a.cells + 3) / 4;
  if (blocks > 65536) blocks = 65536;
  majorant_grid_kernel<<<dim3(unsigned(blocks)), dim3(256), 0, stream>>>(a);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

#elif RDV_FIELD_PART == 1
RDV_GEN_FIELD_DEFINE8(launch_raymarch_generic8, raymarch_generic_kernel, TransmittanceGenArgs)
#elif RDV_FIELD_PART == 2
RDV_GEN_FIELD_DEFINE8(launch_ratiotracking_generic8, ratiotracking_generic_kernel, RatioGenArgs)
#elif RDV_FIELD_PART == 3
RDV_GEN_FIELD_DEFINE8(launch_render_ea_generic8, render_ea_generic_kernel, RenderGenArgs)
#endif  // RDV_FIELD_PART

}  // namespace rdv
