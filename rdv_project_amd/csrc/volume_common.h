// Device helpers shared by the ray kernels (render.hip, volume_profile.hip):
// the unit-box slab test, the 3x3 inverse of a mat4x3's linear part, the voxel
// majorant lookup, and the runtime-shaped extinction / field chain evaluated on
// 32 points of a wave with its launch helper.
#pragma once

#include <mutex>
#include <vector>

#include "mlp_core.h"
#include "mlp_generic.h"

namespace rdv {

// A block's share of the n rays of a launch of G blocks.  Rays are taken in units
// of 32 consecutive rays (one ray each when a block's share is below 256 rays, so
// that small launches still spread over every block); G consecutive units form a
// group, and block b takes unit (b + 37 k) mod G of group k.  Every block thus gets
// rays from every part of a camera image: the work of a ray follows its path
// through the box, and contiguous ranges of image rows gave the blocks at the
// centre of the C4 frame up to 38% more fixed steps than the mean.  A unit keeps
// neighbouring rays together, so the rays a wave claims at once stay coherent.
// Slots of the last group may name rays >= n, which the kernels skip.  With
// spread = false a block takes the contiguous range b ceil(n / G) + k instead (the
// emission-absorption renderer, whose work per ray hardly varies: there the spread
// order measured 2.5% slower).
struct BlockRays {
  int64_t n;
  int g, b, shift;  // shift < 0: contiguous ranges
  int count;        // slots of every block
  __device__ explicit BlockRays(int64_t nrays, bool spread = true)
      : n(nrays), g(int(gridDim.x)), b(int(blockIdx.x)) {
    const int64_t per = (nrays + g - 1) / g;
    if (!spread) {
      shift = -1;
      count = int(per);
      return;
    }
    shift = per >= 256 ? 5 : 0;
    const int64_t unit = int64_t(g) << shift;
    count = int(((nrays + unit - 1) / unit) << shift);
  }
  __device__ int64_t ray(int k) const {
    if (shift < 0) return int64_t(b) * count + k;
    const int64_t grp = k >> shift;
    return ((grp * g + (b + 37 * grp) % g) << shift) + (k & ((1 << shift) - 1));
  }
};

// math_library.h:48-57: slab test against [-1, 1]^3.
// Every operation rounded on its own: a contracted -x * inv +- s moves the exit
// distance by an ulp against the voxel exits computed from the same ray, which
// changes where a tracked ray's last flight ends.
__device__ __forceinline__ void ray_box(const float (&x)[3], const float (&w)[3], float& tmin, float& tmax) {
#pragma clang fp contract(off)
  float c0[3], c1[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const float inv = 1.0f / w[i];
    const float xc = -x[i] * inv;
    const float s = fabsf(inv);
    c0[i] = xc - s;
    c1[i] = xc + s;
  }
  tmin = fmaxf(fmaxf(c0[0], c0[1]), c0[2]);
  tmax = fminf(fminf(c1[0], c1[1]), c1[2]);
}

// GLSL inverse() of the 3x3 linear part by the adjugate (columns c0, c1, c2).
__device__ __forceinline__ void inverse3(const float (&M)[12], float (&L)[9]) {
  const float a00 = M[0], a01 = M[1], a02 = M[2];  // column 0
  const float a10 = M[3], a11 = M[4], a12 = M[5];  // column 1
  const float a20 = M[6], a21 = M[7], a22 = M[8];  // column 2
  const float b01 = a22 * a11 - a12 * a21;
  const float b11 = -a22 * a10 + a12 * a20;
  const float b21 = a21 * a10 - a11 * a20;
  const float det = a00 * b01 + a01 * b11 + a02 * b21;
  const float id = 1.0f / det;
  L[0] = b01 * id;
  L[1] = (-a22 * a01 + a02 * a21) * id;
  L[2] = (a12 * a01 - a02 * a11) * id;
  L[3] = b11 * id;
  L[4] = (a22 * a00 - a02 * a20) * id;
  L[5] = (-a12 * a00 + a02 * a10) * id;
  L[6] = b21 * id;
  L[7] = (-a21 * a00 + a01 * a20) * id;
  L[8] = (a11 * a00 - a01 * a10) * id;
}

constexpr int64_t kGenFieldLdsCap = 152 * 1024;

// A-fragment and bias sources of a block: the LDS copy (staged here) or the
// packed block in global memory.
template <bool LDSW>
__device__ __forceinline__ void gen_sources(const uint8_t* packed, const GenNet& g, uint8_t* smem, const half8** w,
                                            const float** b) {
  if constexpr (LDSW) {
    gen_stage(packed, g, smem);
    *w = reinterpret_cast<const half8*>(smem);
    *b = reinterpret_cast<const float*>(smem + int64_t(g.n_frag) * 1024);
  } else {
    *w = reinterpret_cast<const half8*>(packed + g.frag_off0);
    *b = reinterpret_cast<const float*>(packed + g.bias_off0);
  }
}

// The chain's head value of row 0 at this lane's sample p (3 coordinates).
// F32L: the chain may hold exact fp32 layers (gen_chain_mixed).
template <int MT, bool F32L = false>
__device__ __forceinline__ float gen_field_row0(const GenNet& g, const half8* w0, const float* b0, bool has_bias,
                                                int lane, int h, const float (&p)[3], int act) {
  const int z = opaque_zero();
  const half8* wsrc = w0 + z;
  auto wf = [&](int f) { return wsrc[f * 64 + lane]; };
  auto get = [&](int d) { return d == 0 ? p[0] : (d == 1 ? p[1] : p[2]); };
  float v = 0.0f;
  if constexpr (!F32L && MT >= 2) {
    if (g.fast) {  // GenFieldNet (gen_net checked the shape and layout): the compiled chain
      using N = GenFieldNet;
      const LdsWeights ws{wsrc, lane};
      half8 b[N::kMaxKC];
      f32x16 acc0[N::kMaxMT], acc1[N::kMaxMT];
      build_input<N>(p, h, b);
      if (has_bias) {
        load_bias<N, 0>(acc0, b0 + z, h);
        run_chain<N, 0, true, true>(ws, b, acc0, acc1, b0 + z, h);
      } else {
        run_chain<N, 0, true, false>(ws, b, acc0, acc1, b0, h);
      }
      // the last layer's result is in set (kL - 1) % 2
      return gen_head_act(act, 0, (N::kL - 1) % 2 == 0 ? acc0[0][0] : acc1[0][0]);
    }
  }
  auto sink = [&](const auto& acc) { v = gen_head_act(act, 0, acc[0][0]); };
  if constexpr (F32L) {
    gen_chain_mixed<MT>(g, GenCtx{b0 + z, has_bias, h}, wf, get, sink);
  } else {
    auto l0 = [&](int c) { return gen_l0_chunk(g, c, h, get); };
    gen_chain<MT>(g, GenCtx{b0 + z, has_bias, h}, wf, l0, sink);
  }
  return v;
}

// GenFieldNet's head value at 64 points, one per lane (the 64-ray kernels):
// tile A holds the points of lanes 0-31 and tile B those of lanes 32-63, run as
// a staggered pair (run_pair).  Layer 0 reads 3 features, all in a lane's low
// K half, so lanes 32-63 give zeros to both tiles' B fragments and lanes 0-31
// give tile B the point of lane + 32.  Row 0 of column n is in lane n of each
// tile's D; tile B's goes back to lane n + 32.
__device__ __forceinline__ float gen_field_pair64(const half8* w0, const float* b0, bool has_bias, int lane, int h,
                                                  const float (&p)[3], int act) {
  using N = GenFieldNet;
  const int z = opaque_zero();
  const LdsWeights ws{w0 + z, lane};
  float ps[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) ps[i] = __shfl_xor(p[i], 32);
  half8 bA[N::kMaxKC], bB[N::kMaxKC];
  f32x16 accA[N::kMaxMT], accB[N::kMaxMT];
  build_input<N>(p, h, bA);
  if (has_bias) run_pair<N, 0, true, true>(ws, ps, h, bA, bB, accA, accB, b0 + z);
  else run_pair<N, 0, true, false>(ws, ps, h, bA, bB, accA, accB, b0);
  const float vb = __shfl_xor(accB[0][0], 32);
  return gen_head_act(act, 0, h == 0 ? accA[0][0] : vb);
}

// voxel_majorant_field.h: the majorant of the voxel holding x and the distance
// along w to that voxel's exit.
__device__ __forceinline__ float voxel_majorant(const float* __restrict__ grid, int mw, int mh, int md,
                                                const float (&x)[3], const float (&w)[3], float& dist) {
#pragma clang fp contract(off)
  const int dim[3] = {mw, mh, md};
  int cell[3];
  float te[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const float fd = float(dim[i]);
    // int() truncates toward zero; clamping first keeps the conversion in range
    // (and sends NaN to 0) without changing any in-range result.
    const float f = (x[i] * 0.5f + 0.5f) * fd;
    cell[i] = int(fminf(fmaxf(f, 0.0f), fd - 1.0f));
    const float vs = 2.0f / fd;
    const float bmin = float(cell[i]) * vs - 1.0f;
    const float bmax = bmin + vs;
    const float t0 = (bmin - x[i]) / w[i];
    const float t1 = (bmax - x[i]) / w[i];
    te[i] = fmaxf(t0, t1);
  }
  dist = fminf(fminf(te[0], te[1]), te[2]);
  return grid[(int64_t(cell[2]) * mh + cell[1]) * mw + cell[0]];
}

// Raises `kernel`'s dynamic-LDS limit to kGenFieldLdsCap, once per kernel.
static int gen_field_lds_attr(const void* kernel) {
  static std::mutex mu;
  static std::vector<const void*> done;
  std::lock_guard<std::mutex> lock(mu);
  for (const void* k : done)
    if (k == kernel) return RDV_OK;
  RDV_HIP_TRY(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, int(kGenFieldLdsCap)));
  done.push_back(kernel);
  return RDV_OK;
}

template <class Args, int MT, bool LDSW>
static int launch_gen_field(void (*kernel)(Args), const Args& a, int64_t work_items, int cu, size_t lds,
                            hipStream_t stream) {
  if (LDSW) {
    const int rc = gen_field_lds_attr(reinterpret_cast<const void*>(kernel));
    if (rc != RDV_OK) return rc;
  }
  constexpr int waves = gen_waves<MT>();
  int64_t blocks = cu;
  const int64_t need = (work_items + waves - 1) / waves;
  if (need < blocks) blocks = need;
  kernel<<<dim3(unsigned(blocks)), dim3(64 * waves), lds, stream>>>(a);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

// Launch of a runtime-shaped field kernel KERNEL<MT, LDSW> for NET, with the
// 8-tile instantiations (chains with a layer wider than 128) handed to
// LAUNCH8, defined by RDV_GEN_FIELD_DEFINE8 in a translation unit of its own:
// they take most of a source's compile time, and separate units build in
// parallel.
#define RDV_GEN_FIELD_DISPATCH(KERNEL, ARGS, ITEMS, CU, NET, STREAM, LAUNCH8)                                 \
  do {                                                                                                       \
    const int64_t lds_ = gen_lds_bytes(NET);                                                                 \
    const bool in_lds_ = lds_ <= kGenFieldLdsCap;                                                            \
    switch (gen_mt_bound(NET)) {                                                                             \
      case 1:                                                                                                \
        return in_lds_ ? launch_gen_field<decltype(ARGS), 1, true>(&KERNEL<1, true>, ARGS, ITEMS, CU, lds_, STREAM) \
                       : launch_gen_field<decltype(ARGS), 1, false>(&KERNEL<1, false>, ARGS, ITEMS, CU, 0, STREAM); \
      case 2:                                                                                                \
        return in_lds_ ? launch_gen_field<decltype(ARGS), 2, true>(&KERNEL<2, true>, ARGS, ITEMS, CU, lds_, STREAM) \
                       : launch_gen_field<decltype(ARGS), 2, false>(&KERNEL<2, false>, ARGS, ITEMS, CU, 0, STREAM); \
      case 4:                                                                                                \
        return in_lds_ ? launch_gen_field<decltype(ARGS), 4, true>(&KERNEL<4, true>, ARGS, ITEMS, CU, lds_, STREAM) \
                       : launch_gen_field<decltype(ARGS), 4, false>(&KERNEL<4, false>, ARGS, ITEMS, CU, 0, STREAM); \
      default:                                                                                               \
        return LAUNCH8(ARGS, ITEMS, CU, lds_, in_lds_, STREAM);                                              \
    }                                                                                                        \
  } while (0)

// Definition of the 8-tile launcher LAUNCH8 of KERNEL (arguments ARGS_T).
#define RDV_GEN_FIELD_DEFINE8(LAUNCH8, KERNEL, ARGS_T)                                                       \
  int LAUNCH8(const ARGS_T& a, int64_t items, int cu, int64_t lds, bool in_lds, hipStream_t stream) {        \
    return in_lds ? launch_gen_field<ARGS_T, 8, true>(&KERNEL<8, true>, a, items, cu, lds, stream)           \
                  : launch_gen_field<ARGS_T, 8, false>(&KERNEL<8, false>, a, items, cu, 0, stream);           \
  }

// A LinearFast chain from 3 inputs (raw or FREQ-encoded) to `out` outputs?
static bool is_f16_field(const rdv_mlp_desc& d, int out) {
  if (d.in_features != 3 || d.dims[d.n_layers] != out) return false;
  for (int i = 0; i < d.n_layers; ++i)
    if (d.prec[i] != RDV_PREC_F16) return false;
  return true;
}

// Largest M-tile count of a chain with exact fp32 layers that the field kernels
// instantiate (widths up to 64: the fp32 input blocks held between layers stay
// within the ray kernels' register budget).
constexpr int kGenMixedMaxMT = 2;

// A chain from 3 inputs to `out` outputs with at least one exact fp32 layer,
// whose widths the mixed field kernels take?  Its fragments (fp32 ones are
// twice the bytes of fp16) must fit in the field kernels' LDS.
static bool is_mixed_field(const rdv_mlp_desc& d, const MlpLayout& lay, int out, std::string* why) {
  if (d.in_features != 3 || d.dims[d.n_layers] != out) return false;
  bool any = false;
  for (int i = 0; i < d.n_layers; ++i) any = any || d.prec[i] == RDV_PREC_F32;
  if (!any) return false;
  GenNet g;
  gen_net(d, lay, &g);
  if (g.max_mt > kGenMixedMaxMT) {
    *why = "a field chain with exact fp32 (Linear) layers supports widths up to " + std::to_string(32 * kGenMixedMaxMT);
    return false;
  }
  if (gen_lds_bytes(g) > kGenFieldLdsCap) {
    *why = "a field chain with exact fp32 (Linear) layers must fit in " + std::to_string(kGenFieldLdsCap / 1024) +
           " KiB of fragments and biases";
    return false;
  }
  return true;
}

template <class Args, int MT>
static int launch_gen_field_mixed(void (*kernel)(Args), const Args& a, int64_t work_items, int cu, size_t lds,
                                  hipStream_t stream) {
  return launch_gen_field<Args, MT, true>(kernel, a, work_items, cu, lds, stream);
}

// Launch of KERNEL<MT, true, true> (weights in LDS, exact fp32 layers) for NET.
#define RDV_GEN_FIELD_DISPATCH_MIXED(KERNEL, ARGS, ITEMS, CU, NET, STREAM)                                  \
  do {                                                                                                      \
    const int64_t lds_ = gen_lds_bytes(NET);                                                                \
    if (gen_mt_bound(NET) == 1)                                                                             \
      return launch_gen_field_mixed<decltype(ARGS), 1>(&KERNEL<1, true, true>, ARGS, ITEMS, CU, lds_, STREAM); \
    return launch_gen_field_mixed<decltype(ARGS), 2>(&KERNEL<2, true, true>, ARGS, ITEMS, CU, lds_, STREAM);   \
  } while (0)

}  // namespace rdv
