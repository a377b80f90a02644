// Per-layer tensor operations: y[rows, out] = x[rows, in] W^T + b and
// y = max(x, 0), one dispatch per op, fp32 buffers in and out.
//
// Reference: the TensorOperation family (src/rdv/maths/__init__.py:1251-1380),
//   LinearTensorOp       src/rdv/shaders/tensors/linear_tensor_op.h:8-51       (fp32)
//   LinearTensorOpSmall  src/rdv/shaders/tensors/linear_tensor_op_small.h:50-247 (fp16 x, W; fp32 acc)
//   LinearTensorOpSimple src/rdv/shaders/tensors/linear_tensor_op_simple.h:49-116
//   LinearTensorOpFast   src/rdv/shaders/tensors/linear_tensor_op_fast.h:37-122
//   LinearTensorOpMine   src/rdv/shaders/tensors/linear_tensor_op_mine.h:51-133
//   ReLUTensorOp         src/rdv/shaders/tensors/relu_tensor_op.h:3-22
// The four fp16 variants compute the same function (x and W rounded to fp16,
// products accumulated in fp32, fp32 bias) and differ only in tiling, so one
// kernel serves them; the weight may arrive as fp32 [out, in] (read and rounded
// at dispatch, like Small and Mine), fp16 [out, in] (Simple's pre-cast copy) or
// fp16 [out/16][in/16][16 k][16 n] tiles (Fast's pre-tiled copy, nn.py:472-490).
//
// MI355X mapping.  The op is streaming: at in = out = 128 it does 32 flops per
// HBM byte against a ridge of ~300, so the bound is HBM and the design goal is
// to touch every x and y byte once with wide accesses while the whole weight
// block sits in LDS.  Each workgroup (4 waves) owns one block of <= 128 outputs
// for the whole run: it stages that block of W (and of the bias) into LDS once,
// in MFMA-fragment order, then walks row tiles with a grid stride and no further
// barrier.  A wave computes D^T = W x^T for 16-row subtiles:
//   fp16: v_mfma_f32_16x16x32_f16, A = W[16 out][32 k], B = x^T[32 k][16 rows];
//         lane (r = l%16, q = l/16) loads x[r][8q..8q+7] as two 16-byte loads.
//   fp32: v_mfma_f32_16x16x4f32 over 16-k groups; lane (r, q) loads x[r][4q..4q+3]
//         once and feeds one element to each of 4 MFMAs (MFMA k index q stands
//         for k = 4q + s in step s; W fragments are staged in the same order).
//   D[out 4q+j][row r] leaves each lane with 4 consecutive outputs of one row:
//   one 16-byte store per (subtile, out tile).  Loads and stores are ordinary
//   (cached): each instruction covers only half of every 128-byte line it
//   touches, and with non-temporal hints the halves reach HBM separately
//   (measured: 20% more bytes written and 16% lower throughput at 128 -> 128).
// The next tile's x loads are issued right after the current tile's loads have
// been converted, so they stream under the MFMAs and stores.  When in exceeds
// one LDS pass (256 fp16 / 128 fp32 columns) the weight is restaged per pass and
// per tile instead (a plain tiled GEMM).
#include <algorithm>

#include "rdv_common.h"

namespace rdv {

namespace {

constexpr int kLoThreads = 256;
constexpr int kLoWaves = kLoThreads / 64;
constexpr int kLoMaxOb = 128;  // outputs per workgroup block

struct LinearOpArgs {
  const float* x;     // [rows, in]
  const void* w;      // weight (wkind)
  const float* bias;  // [out]
  float* y;           // [rows, out]
  int64_t rows;
  int64_t tasks;      // row tiles of kLoWaves * 16 * RT rows
  int in, out;
  int wkind;          // RDV_WKIND_*
  int relu;
  int kp;             // columns of x per LDS pass (multiple of the k step)
  int passes;         // ceil(in / kp)
  int ob;             // outputs per block (multiple of 16)
  int n_ob;           // ceil(out / ob)
};

// One k chunk of one lane: F16 -> 8 columns (two float4), F32 -> 4 columns.
template <bool F16>
struct LoPolicy;
template <>
struct LoPolicy<true> {
  static constexpr int kStep = 32;  // columns per chunk
  static constexpr int kVec = 2;    // float4 loads per lane per chunk
};
template <>
struct LoPolicy<false> {
  static constexpr int kStep = 16;
  static constexpr int kVec = 1;
};

__device__ __forceinline__ half8 to_half8(f32x4 a, f32x4 b) {
  half8 h;
  h[0] = half_t(a[0]); h[1] = half_t(a[1]); h[2] = half_t(a[2]); h[3] = half_t(a[3]);
  h[4] = half_t(b[0]); h[5] = half_t(b[1]); h[6] = half_t(b[2]); h[7] = half_t(b[3]);
  return h;
}

// Stages outputs [o0, o0 + ob) x columns [k0, k0 + kp) of W into LDS in fragment
// order: slot ((t * nkc + c) * 64 + lane) holds 16 bytes, W[o0 + 16t + lane%16]
// [k0 + c*kStep + (lane/16)*(kStep/4) ...] as 8 halves (fp16) or 4 floats (fp32).
// Rows past `out` and columns past `in` are zero.  Also stages the bias block.
template <bool F16>
__device__ void stage_weight(const LinearOpArgs& a, int o0, int k0, int nkc, f32x4* sw, float* sb) {
  using P = LoPolicy<F16>;
  const int nt = a.ob / 16;
  const int slots = nt * nkc * 64;
  for (int s = threadIdx.x; s < slots; s += kLoThreads) {
    const int t = s / (nkc * 64);
    const int rem = s - t * (nkc * 64);
    const int c = rem >> 6;
    const int ln = rem & 63;
    const int o = o0 + 16 * t + (ln & 15);
    const int k = k0 + c * P::kStep + (ln >> 4) * (P::kStep / 4);
    const bool ok = o < a.out && k < a.in;
    f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if (ok) {
      if constexpr (F16) {
        half8 h;
        if (a.wkind == RDV_WKIND_F32) {
          const f32x4* src = reinterpret_cast<const f32x4*>(static_cast<const float*>(a.w) + int64_t(o) * a.in + k);
          h = to_half8(src[0], src[1]);
        } else if (a.wkind == RDV_WKIND_F16) {
          h = *reinterpret_cast<const half8*>(static_cast<const half_t*>(a.w) + int64_t(o) * a.in + k);
        } else {  // fp16 tiles [out/16][in/16][16 k][16 n]
          const half_t* wt = static_cast<const half_t*>(a.w);
          const int64_t base = (int64_t(o >> 4) * (a.in >> 4) + (k >> 4)) * 256 + (o & 15);
#pragma unroll
          for (int i = 0; i < 8; ++i) h[i] = wt[base + ((k & 15) + i) * 16];
        }
        v = __builtin_bit_cast(f32x4, h);
      } else {
        v = *reinterpret_cast<const f32x4*>(static_cast<const float*>(a.w) + int64_t(o) * a.in + k);
      }
    }
    sw[s] = v;
  }
  for (int i = threadIdx.x; i < a.ob; i += kLoThreads) sb[i] = (o0 + i < a.out) ? a.bias[o0 + i] : 0.0f;
}

// Loads one wave's x for row tile `task`, columns [k0, k0 + NKC*kStep): raw[rr][c][v].
// Rows are clamped into range (their results are never stored) and columns past
// `in` are clamped to column 0 (zeroed on conversion), so every load is in bounds
// and unconditional.
template <bool F16, int RT, int NKC>
__device__ __forceinline__ void load_x(const LinearOpArgs& a, int64_t task, int k0, int nkc, int wave, int lane,
                                       f32x4 (&raw)[RT][NKC][LoPolicy<F16>::kVec]) {
  using P = LoPolicy<F16>;
  const int q = lane >> 4;
#pragma unroll
  for (int rr = 0; rr < RT; ++rr) {
    int64_t row = (task * kLoWaves + wave) * (16 * RT) + rr * 16 + (lane & 15);
    row = row < a.rows ? row : a.rows - 1;
    const float* xr = a.x + row * a.in;
#pragma unroll
    for (int c = 0; c < NKC; ++c) {
      if (c >= nkc) break;  // nkc is uniform: a scalar branch
      int k = k0 + c * P::kStep + q * (P::kStep / 4);
      k = k < a.in ? k : 0;
#pragma unroll
      for (int v = 0; v < P::kVec; ++v) raw[rr][c][v] = reinterpret_cast<const f32x4*>(xr + k)[v];
    }
  }
}

template <bool F16, int RT, int NKC>
struct XFrag;
template <int RT, int NKC>
struct XFrag<true, RT, NKC> {
  half8 v[RT][NKC];
};
template <int RT, int NKC>
struct XFrag<false, RT, NKC> {
  f32x4 v[RT][NKC];
};

template <bool F16, int RT, int NKC>
__device__ __forceinline__ void convert_x(const LinearOpArgs& a, int k0, int nkc, int lane,
                                          const f32x4 (&raw)[RT][NKC][LoPolicy<F16>::kVec],
                                          XFrag<F16, RT, NKC>& xf) {
  using P = LoPolicy<F16>;
  const int q = lane >> 4;
#pragma unroll
  for (int c = 0; c < NKC; ++c) {
    const bool ok = c < nkc && k0 + c * P::kStep + q * (P::kStep / 4) < a.in;
#pragma unroll
    for (int rr = 0; rr < RT; ++rr) {
      if constexpr (F16) {
        const half8 h = to_half8(raw[rr][c][0], raw[rr][c][1]);
        xf.v[rr][c] = ok ? h : half8{};
      } else {
        xf.v[rr][c] = ok ? raw[rr][c][0] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
  }
}

template <bool F16, int RT, int NKC>
__device__ __forceinline__ void mma_pass(const f32x4* sw, int nt, int nkc, int lane, const XFrag<F16, RT, NKC>& xf,
                                         f32x4 (&acc)[RT][kLoMaxOb / 16]) {
#pragma unroll
  for (int t = 0; t < kLoMaxOb / 16; ++t) {
    if (t < nt) {
#pragma unroll
      for (int c = 0; c < NKC; ++c) {
        if (c < nkc) {
          const f32x4 wv = sw[(t * nkc + c) * 64 + lane];
          if constexpr (F16) {
            const half8 wh = __builtin_bit_cast(half8, wv);
#pragma unroll
            for (int rr = 0; rr < RT; ++rr)
              acc[rr][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wh, xf.v[rr][c], acc[rr][t], 0, 0, 0);
          } else {
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
              for (int rr = 0; rr < RT; ++rr)
                acc[rr][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[s], xf.v[rr][c][s], acc[rr][t], 0, 0, 0);
          }
        }
      }
    }
  }
}

template <int RT>
__device__ __forceinline__ void seed_bias(const float* sb, int nt, int lane, f32x4 (&acc)[RT][kLoMaxOb / 16]) {
  const f32x4* sb4 = reinterpret_cast<const f32x4*>(sb);
#pragma unroll
  for (int t = 0; t < kLoMaxOb / 16; ++t) {
    const f32x4 b = t < nt ? sb4[t * 4 + (lane >> 4)] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int rr = 0; rr < RT; ++rr) acc[rr][t] = b;
  }
}

template <int RT>
__device__ __forceinline__ void store_y(const LinearOpArgs& a, int64_t task, int o0, int nt, int wave, int lane,
                                        const f32x4 (&acc)[RT][kLoMaxOb / 16]) {
#pragma unroll
  for (int rr = 0; rr < RT; ++rr) {
    const int64_t row = (task * kLoWaves + wave) * (16 * RT) + rr * 16 + (lane & 15);
    if (row < a.rows) {
      float* yr = a.y + row * a.out;
#pragma unroll
      for (int t = 0; t < kLoMaxOb / 16; ++t) {
        const int col = o0 + 16 * t + 4 * (lane >> 4);
        if (t < nt && col < a.out) {
          f32x4 v = acc[rr][t];
          if (a.relu) {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = fmaxf(v[j], 0.0f);
          }
          *reinterpret_cast<f32x4*>(yr + col) = v;
        }
      }
    }
  }
}

template <bool F16, int RT, int NKC>
__global__ __launch_bounds__(kLoThreads) void linear_op_kernel(LinearOpArgs a) {
  using P = LoPolicy<F16>;
  extern __shared__ f32x4 lo_smem[];
  const int nt = a.ob / 16;
  const int nkc = (a.kp + P::kStep - 1) / P::kStep;
  f32x4* sw = lo_smem;
  float* sb = reinterpret_cast<float*>(lo_smem + nt * nkc * 64);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // blockIdx.x = row workgroup * n_ob + output block: the blocks sharing rows
  // are dispatched back to back, so their x re-reads hit the shared cache.
  const int ob_idx = blockIdx.x % a.n_ob;
  const int64_t rwg = blockIdx.x / a.n_ob;
  const int64_t rstride = gridDim.x / a.n_ob;
  const int o0 = ob_idx * a.ob;

  f32x4 raw[RT][NKC][P::kVec];
  XFrag<F16, RT, NKC> xf;
  f32x4 acc[RT][kLoMaxOb / 16];

  if (a.passes == 1) {
    stage_weight<F16>(a, o0, 0, nkc, sw, sb);
    __syncthreads();
    int64_t task = rwg;
    if (task >= a.tasks) return;
    load_x<F16, RT, NKC>(a, task, 0, nkc, wave, lane, raw);
    for (; task < a.tasks; task += rstride) {
      convert_x<F16, RT, NKC>(a, 0, nkc, lane, raw, xf);
      int64_t next = task + rstride;
      next = next < a.tasks ? next : a.tasks - 1;
      load_x<F16, RT, NKC>(a, next, 0, nkc, wave, lane, raw);
      seed_bias<RT>(sb, nt, lane, acc);
      mma_pass<F16, RT, NKC>(sw, nt, nkc, lane, xf, acc);
      store_y<RT>(a, task, o0, nt, wave, lane, acc);
    }
    return;
  }

  // in > one pass: restage W per pass and per tile.
  for (int64_t task = rwg; task < a.tasks; task += rstride) {
    for (int p = 0; p < a.passes; ++p) {
      const int k0 = p * a.kp;
      __syncthreads();
      stage_weight<F16>(a, o0, k0, nkc, sw, sb);
      __syncthreads();
      if (p == 0) seed_bias<RT>(sb, nt, lane, acc);
      load_x<F16, RT, NKC>(a, task, k0, nkc, wave, lane, raw);
      convert_x<F16, RT, NKC>(a, k0, nkc, lane, raw, xf);
      mma_pass<F16, RT, NKC>(sw, nt, nkc, lane, xf, acc);
    }
    store_y<RT>(a, task, o0, nt, wave, lane, acc);
  }
}

__global__ __launch_bounds__(256) void relu_op_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
  const int64_t n4 = n >> 2;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  const f32x4* x4 = reinterpret_cast<const f32x4*>(x);
  f32x4* y4 = reinterpret_cast<f32x4*>(y);
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
    f32x4 v = __builtin_nontemporal_load(x4 + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = fmaxf(v[j], 0.0f);
    __builtin_nontemporal_store(v, y4 + i);
  }
  const int64_t t = (n4 << 2) + int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (blockIdx.x == 0 && t < n) y[t] = fmaxf(x[t], 0.0f);
}

struct LoKernel {
  const void* fn;
  int rt;
  int occupancy;  // resident workgroups per CU (0 = not yet queried)
};

template <bool F16, int RT, int NKC>
const void* lo_fn() {
  return reinterpret_cast<const void*>(&linear_op_kernel<F16, RT, NKC>);
}

}  // namespace

int linear_op_check(const rdv_linear_op_desc& d, std::string* why) {
  auto bad = [&](const std::string& m) {
    *why = m;
    return RDV_ERR_INVALID;
  };
  if (d.rows < 0) return bad("rows must be >= 0");
  if (d.precision != RDV_PREC_F16 && d.precision != RDV_PREC_F32) return bad("unknown precision code");
  if (d.wkind != RDV_WKIND_F32 && d.wkind != RDV_WKIND_F16 && d.wkind != RDV_WKIND_F16_TILED16)
    return bad("unknown weight kind");
  if (d.precision == RDV_PREC_F32 && d.wkind != RDV_WKIND_F32)
    return bad("fp32 precision needs an fp32 weight");
  if (d.in_features < 8 || d.in_features % 8)
    return bad("in_features (" + std::to_string(d.in_features) + ") must be a positive multiple of 8");
  if (d.out_features < 4 || d.out_features % 4)
    return bad("out_features (" + std::to_string(d.out_features) + ") must be a positive multiple of 4");
  if (d.wkind == RDV_WKIND_F16_TILED16 && (d.in_features % 16 || d.out_features % 16))
    return bad("tiled fp16 weights need in_features and out_features multiples of 16");
  if (int64_t(d.in_features) * d.out_features >= (int64_t(1) << 31)) return bad("weight too large");
  if (d.rows >= (int64_t(1) << 40)) return bad("too many rows");
  return RDV_OK;
}

int launch_linear_op(const rdv_linear_op_desc& d, const float* x, const void* w, const float* bias, float* y,
                     hipStream_t stream) {
  if (d.rows == 0) return RDV_OK;
  DeviceInfo dev;
  if (int rc = device_info(&dev)) return rc;
  const bool f16 = d.precision == RDV_PREC_F16;
  const int step = f16 ? 32 : 16;
  const int kmax = f16 ? 256 : 128;
  const int chunks = (d.in_features + step - 1) / step;
  const int passes = (d.in_features + kmax - 1) / kmax;
  const int per_pass = (chunks + passes - 1) / passes;
  int nkc = 1;
  while (nkc < per_pass) nkc *= 2;
  const int rt = nkc <= 4 ? 2 : 1;

  static LoKernel table[2][4] = {};  // [f16][log2 nkc]
  int li = 0;
  while ((1 << li) < nkc) ++li;
  LoKernel& k = table[f16][li];
  if (!k.fn) {
    const void* fns[2][4] = {
        {lo_fn<false, 2, 1>(), lo_fn<false, 2, 2>(), lo_fn<false, 2, 4>(), lo_fn<false, 1, 8>()},
        {lo_fn<true, 2, 1>(), lo_fn<true, 2, 2>(), lo_fn<true, 2, 4>(), lo_fn<true, 1, 8>()}};
    k.fn = fns[f16][li];
    k.rt = rt;
  }

  LinearOpArgs a;
  a.x = x;
  a.w = w;
  a.bias = bias;
  a.y = y;
  a.rows = d.rows;
  a.in = d.in_features;
  a.out = d.out_features;
  a.wkind = d.wkind;
  a.relu = d.relu ? 1 : 0;
  a.passes = passes;
  a.kp = passes == 1 ? chunks * step : kmax;
  a.ob = std::min(kLoMaxOb, (d.out_features + 15) / 16 * 16);
  a.n_ob = (d.out_features + a.ob - 1) / a.ob;
  const int64_t rows_per_task = int64_t(kLoWaves) * 16 * rt;
  a.tasks = (d.rows + rows_per_task - 1) / rows_per_task;

  const int nkc_run = (a.kp + step - 1) / step;
  const size_t lds = size_t(a.ob / 16) * nkc_run * 64 * sizeof(f32x4) + size_t(a.ob) * sizeof(float);
  if (lds > 64 * 1024 + kLoMaxOb * sizeof(float)) return fail(RDV_ERR_UNSUPPORTED, "linear op LDS plan too large");
  if (!k.occupancy) {
    RDV_HIP_TRY(hipFuncSetAttribute(k.fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    64 * 1024 + kLoMaxOb * int(sizeof(float))));
  }
  int occ = 0;
  RDV_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k.fn, kLoThreads, lds));
  occ = std::max(occ, 1);
  k.occupancy = occ;
  const int64_t slots = int64_t(dev.cu_count) * occ;
  const int64_t rwgs = std::max<int64_t>(1, std::min<int64_t>(a.tasks, (slots + a.n_ob - 1) / a.n_ob));
  const int64_t grid = rwgs * a.n_ob;
  if (grid > 0x7fffffff) return fail(RDV_ERR_UNSUPPORTED, "grid too large");
  void* params[] = {&a};
  RDV_HIP_TRY(hipLaunchKernel(k.fn, dim3(static_cast<unsigned>(grid)), dim3(kLoThreads), params, lds, stream));
  return RDV_OK;
}

int launch_relu_op(const float* x, float* y, int64_t n, hipStream_t stream) {
  if (n == 0) return RDV_OK;
  DeviceInfo dev;
  if (int rc = device_info(&dev)) return rc;
  const int64_t n4 = std::max<int64_t>(1, n >> 2);
  const int64_t blocks = std::min<int64_t>((n4 + 255) / 256, int64_t(dev.cu_count) * 8);
  hipLaunchKernelGGL(relu_op_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, x, y, n);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

}  // namespace rdv
