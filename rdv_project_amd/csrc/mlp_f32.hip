// Chain kernels on the vector ALUs: one thread's arithmetic per row and output.
//
// This is the reference's per-thread evaluation order made explicit:
//  - Linear (src/rdv/shaders/maps/linear.h:36-43):  acc = b[o]; acc += x[k] * W[o][k]
//  - LinearFast on a partial workgroup (linear_fast.h:102-108): the same fp32 loop
//  - LinearFast on a full workgroup (linear_fast.h:61-98) emulated exactly as
//    written: x and W rounded to fp16, products summed in fp32 from zero, then
//    the fp32 bias added.
// It serves chains containing an fp32 Linear layer, shapes without a matrix-core
// instantiation, and the < 32-row tail group that the reference evaluates in fp32.
#include "mlp_layout.h"
#include "rdv_common.h"

namespace rdv {

struct ChainF32Args {
  const float* x;
  float* y;
  const uint8_t* packed;
  int64_t row0;   // first row handled by this launch
  int64_t nrows;  // rows handled by this launch
  int stride;     // LDS row stride in floats (max width + 1)
  int force_f32;  // evaluate F16 layers with the exact fp32 loop (partial-group rule)
  int encoding, enc_d, enc_l;
  int act[RDV_MLP_MAX_LAYERS];
  int prec[RDV_MLP_MAX_LAYERS];
  int direct;        // 1: parameters from dw (the layers' own fp32 buffers), not the packed block
  DirectWeights dw;
  MlpLayout lay;
};

__global__ __launch_bounds__(64) void mlp_chain_f32_kernel(ChainF32Args a) {
  extern __shared__ float lds[];
  const int tid = threadIdx.x;
  const int64_t r = int64_t(blockIdx.x) * 64 + tid;
  const bool live = r < a.nrows;
  const int64_t row = a.row0 + r;
  float* buf0 = lds + tid * a.stride;
  float* buf1 = lds + (64 + tid) * a.stride;

  // layer-0 input (encoded if requested), zero padded to dims[0]
  const int in0 = a.lay.in_w[0];
  const int D = a.enc_d;
  if (live) {
    const float* xr = a.x + row * D;
    if (a.encoding == RDV_ENC_FREQ) {
      for (int d = 0; d < D; ++d) buf0[d] = xr[d];
      for (int k = 0; k < a.enc_l; ++k)
        for (int d = 0; d < D; ++d) {
          const float t = ldexpf(xr[d], k);  // 2^k p, exact
          buf0[D + 2 * D * k + d] = sinpif(t);
          buf0[D + 2 * D * k + D + d] = cospif(t);
        }
      for (int f = D * (1 + 2 * a.enc_l); f < in0; ++f) buf0[f] = 0.0f;
    } else {
      for (int f = 0; f < in0; ++f) buf0[f] = f < D ? xr[f] : 0.0f;
    }
  }

  float* cur = buf0;
  float* nxt = buf1;
  for (int li = 0; li < a.lay.n_layers; ++li) {
    const int iw = a.lay.in_w[li], ow = a.lay.out_w[li];
    const float* __restrict__ W =
        a.direct ? a.dw.W[li] : reinterpret_cast<const float*>(a.packed + a.lay.w32_off[li]);
    const float* __restrict__ B =
        a.direct ? a.dw.b[li] : reinterpret_cast<const float*>(a.packed + a.lay.b32_off[li]);
    const bool f16 = a.prec[li] == RDV_PREC_F16 && !a.force_f32;
    const int act = a.act[li];
    if (live) {
      for (int o = 0; o < ow; ++o) {
        const float* wr = W + int64_t(o) * iw;
        float acc;
        if (f16) {
          acc = 0.0f;
          for (int k = 0; k < iw; ++k) acc = fmaf(float(half_t(cur[k])), float(half_t(wr[k])), acc);
          acc += B[o];
        } else {
          acc = B[o];
          for (int k = 0; k < iw; ++k) acc = fmaf(cur[k], wr[k], acc);
        }
        nxt[o] = apply_act(act, o, acc);
      }
    }
    float* t = cur;
    cur = nxt;
    nxt = t;
  }
  if (live) {
    const int ow = a.lay.out_w[a.lay.n_layers - 1];
    float* yr = a.y + row * ow;
    for (int o = 0; o < ow; ++o) yr[o] = cur[o];
  }
}

// ------------------------------------------------------------ register rows
// The same arithmetic, per output, in the same order, for chains whose widths
// are all at most 64 and whose weights fit in LDS beside the activations:
//  - persistent blocks of 8 waves (two per SIMD); 2 row groups of 128 rows, two
//    rows per lane (r and r + 64), and in each group 4 waves splitting a
//    layer's outputs (o = 4j + og);
//  - a lane's two layer inputs sit in 2 x 64 registers and its weights are read
//    from LDS as 16-byte broadcasts (one address per wave), each weight serving
//    both rows: a broadcast still returns 16 bytes to every lane, so the LDS
//    return path, not the FMAs, bounds a one-row-per-lane layout;
//  - a layer's outputs go through LDS to the group's 4 waves (two barriers).
constexpr int kF32RegWaves = 8;
constexpr int kF32RegGroups = kF32RegWaves / 4;
constexpr int kF32RegRows = 128 * kF32RegGroups;  // rows per block and iteration
constexpr int kF32RegWidth = 64;
// Rows of the activation buffer: 16-byte aligned, so a layer's inputs come back as 16 ds_read_b128 per row
// (lane rows 272 bytes apart: every 16 lanes cover all 64 banks, the full rate of a 16-byte read).
constexpr int kF32RegActStride = kF32RegWidth + 4;

struct ChainF32RegArgs {
  const float* x;
  float* y;
  const uint8_t* packed;
  int64_t row0, nrows;
  int L;
  int encoding, enc_d, enc_l;
  int in_w[RDV_MLP_MAX_LAYERS], out_w[RDV_MLP_MAX_LAYERS];
  int act[RDV_MLP_MAX_LAYERS];
  int f16[RDV_MLP_MAX_LAYERS];   // LinearFast emulation (fp16 operands, sum from zero, bias last)
  int woff[RDV_MLP_MAX_LAYERS];  // LDS float offset of layer l's weights, rows of wstride floats
  int wstride[RDV_MLP_MAX_LAYERS];
  int boff[RDV_MLP_MAX_LAYERS];  // LDS float offset of layer l's bias
  int w_floats;                  // floats of the weight and bias area
  int direct;
  DirectWeights dw;
  MlpLayout lay;
};

// Output o of two rows (inputs c0, c1) in the reference's order (Linear:
// acc = b; acc += x[k] * W[o][k]; LinearFast: products of fp16 operands summed
// from zero, then the bias; the caller has rounded c0 / c1), KQ = ceil(iw / 4)
// 16-byte weight reads.
template <int KQ, bool F16>
__device__ __forceinline__ void f32reg_dot(const float (&c0)[kF32RegWidth], const float (&c1)[kF32RegWidth],
                                           const float* wr, int iw, float bias, float& out0, float& out1) {
  float a0 = F16 ? 0.0f : bias, a1 = F16 ? 0.0f : bias;
#pragma unroll
  for (int q = 0; q < KQ; ++q) {
    const f32x4 w = *reinterpret_cast<const f32x4*>(wr + 4 * q);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = 4 * q + j;
      float t0, t1;
      if constexpr (F16) {  // c0 / c1 already rounded to fp16 by the caller
        const float wh = float(half_t(w[j]));
        t0 = fmaf(c0[k], wh, a0);
        t1 = fmaf(c1[k], wh, a1);
      } else {
        t0 = fmaf(c0[k], w[j], a0);
        t1 = fmaf(c1[k], w[j], a1);
      }
      const bool in = q + 1 < KQ || k < iw;
      a0 = in ? t0 : a0;
      a1 = in ? t1 : a1;
    }
  }
  out0 = F16 ? a0 + bias : a0;
  out1 = F16 ? a1 + bias : a1;
}

// Layer l for the lane's two rows; outputs to dst0 / dst1 (null: not stored).
template <int KQ, bool F16>
__device__ __forceinline__ void f32reg_layer(const ChainF32RegArgs& a, int l, const float (&c0)[kF32RegWidth],
                                             const float (&c1)[kF32RegWidth], const float* sW, float* dst0,
                                             float* dst1, int og) {
  const int iw = a.in_w[l], ow = a.out_w[l], act = a.act[l];
  const float* W = sW + a.woff[l];
  const float* B = sW + a.boff[l];
  const int ws = a.wstride[l];
#pragma nounroll
  for (int o = og; o < ow; o += 4) {
    float v0, v1;
    f32reg_dot<KQ, F16>(c0, c1, W + o * ws, iw, B[o], v0, v1);
    if (dst0 != nullptr) dst0[o] = apply_act(act, o, v0);
    if (dst1 != nullptr) dst1[o] = apply_act(act, o, v1);
  }
}

// Layer-0 input of one row (encoded if requested, zero padded to in0) into act_row.
__device__ __forceinline__ void f32reg_input(const ChainF32RegArgs& a, int64_t row, float* act_row) {
  const int in0 = a.in_w[0], D = a.enc_d;
  const float* xr = a.x + row * D;
  if (a.encoding == RDV_ENC_FREQ) {
    for (int d = 0; d < D; ++d) act_row[d] = xr[d];
    for (int k = 0; k < a.enc_l; ++k)
      for (int d = 0; d < D; ++d) {
        const float t = ldexpf(xr[d], k);  // 2^k p, exact
        act_row[D + 2 * D * k + d] = sinpif(t);
        act_row[D + 2 * D * k + D + d] = cospif(t);
      }
    for (int f = D * (1 + 2 * a.enc_l); f < in0; ++f) act_row[f] = 0.0f;
  } else {
    for (int f = 0; f < in0; ++f) act_row[f] = f < D ? xr[f] : 0.0f;
  }
}

__global__ __launch_bounds__(64 * kF32RegWaves, 1) void mlp_chain_f32_reg_kernel(ChainF32RegArgs a) {
  extern __shared__ __attribute__((aligned(16))) float smem_f32[];
  float* const sW = smem_f32;
  float* const sAct = smem_f32 + a.w_floats;  // [kF32RegGroups][128 rows][kF32RegActStride]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rg = wave >> 2, og = wave & 3;

  // weights (rows padded to wstride, zeros in the padding) and biases into LDS
  for (int l = 0; l < a.L; ++l) {
    const float* W = a.direct ? a.dw.W[l] : reinterpret_cast<const float*>(a.packed + a.lay.w32_off[l]);
    const float* B = a.direct ? a.dw.b[l] : reinterpret_cast<const float*>(a.packed + a.lay.b32_off[l]);
    const int iw = a.in_w[l], ow = a.out_w[l], ws = a.wstride[l];
    if (iw == ws && (reinterpret_cast<uintptr_t>(W) & 15) == 0) {  // rows of whole quartets: a float4 copy
      const f32x4* W4 = reinterpret_cast<const f32x4*>(W);
      f32x4* d4 = reinterpret_cast<f32x4*>(sW + a.woff[l]);
      for (int i = threadIdx.x; i < ow * iw / 4; i += blockDim.x) d4[i] = W4[i];
    } else {
      for (int i = threadIdx.x; i < ow * ws; i += blockDim.x) {
        const int o = i / ws, k = i - o * ws;
        sW[a.woff[l] + i] = k < iw ? W[int64_t(o) * iw + k] : 0.0f;
      }
    }
    for (int i = threadIdx.x; i < ow; i += blockDim.x) sW[a.boff[l] + i] = B[i];
  }
  __syncthreads();

  float* const act0 = sAct + (rg * 128 + lane) * kF32RegActStride;
  float* const act1 = act0 + 64 * kF32RegActStride;
  for (int64_t base = int64_t(blockIdx.x) * kF32RegRows; base < a.nrows; base += int64_t(gridDim.x) * kF32RegRows) {
    const int64_t r0 = base + rg * 128 + lane, r1 = r0 + 64;
    const bool live0 = r0 < a.nrows, live1 = r1 < a.nrows;
    const int64_t row0 = a.row0 + (live0 ? r0 : a.nrows - 1);
    const int64_t row1 = a.row0 + (live1 ? r1 : a.nrows - 1);
    if (og == 0) {  // the group's first wave writes the layer-0 inputs
      f32reg_input(a, row0, act0);
      f32reg_input(a, row1, act1);
    }
    __syncthreads();
    for (int l = 0; l < a.L; ++l) {
      float c0[kF32RegWidth], c1[kF32RegWidth];
#pragma unroll
      for (int q = 0; q < kF32RegWidth / 4; ++q) {
        const f32x4 v0 = *reinterpret_cast<const f32x4*>(act0 + 4 * q);
        const f32x4 v1 = *reinterpret_cast<const f32x4*>(act1 + 4 * q);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          c0[4 * q + j] = v0[j];
          c1[4 * q + j] = v1[j];
        }
      }
      __syncthreads();  // every wave of the group holds the layer input before it is overwritten
      const bool last = l + 1 == a.L;
      float* d0 = last ? (live0 ? a.y + row0 * a.out_w[l] : nullptr) : act0;
      float* d1 = last ? (live1 ? a.y + row1 * a.out_w[l] : nullptr) : act1;
      const int kq = (a.in_w[l] + 3) >> 2;
      const bool f16 = a.f16[l] != 0;
      if (f16) {  // a LinearFast layer's inputs in fp16, rounded once for all of its outputs
#pragma unroll
        for (int k = 0; k < kF32RegWidth; ++k) {
          c0[k] = float(half_t(c0[k]));
          c1[k] = float(half_t(c1[k]));
        }
      }
#define RDV_F32REG(KQ) \
  if (f16) f32reg_layer<KQ, true>(a, l, c0, c1, sW, d0, d1, og); else f32reg_layer<KQ, false>(a, l, c0, c1, sW, d0, d1, og)
      switch (kq) {
        case 1: RDV_F32REG(1); break;
        case 2: RDV_F32REG(2); break;
        case 3: RDV_F32REG(3); break;
        case 4: RDV_F32REG(4); break;
        case 5: RDV_F32REG(5); break;
        case 6: RDV_F32REG(6); break;
        case 7: RDV_F32REG(7); break;
        case 8: RDV_F32REG(8); break;
        case 9: RDV_F32REG(9); break;
        case 10: RDV_F32REG(10); break;
        case 11: RDV_F32REG(11); break;
        case 12: RDV_F32REG(12); break;
        case 13: RDV_F32REG(13); break;
        case 14: RDV_F32REG(14); break;
        case 15: RDV_F32REG(15); break;
        default: RDV_F32REG(16); break;
      }
#undef RDV_F32REG
      __syncthreads();  // the layer's outputs are in LDS for the group
    }
  }
}

static size_t chain_lds_bytes(const rdv_mlp_desc& d) {
  int maxw = 0;
  for (int i = 0; i <= d.n_layers; ++i) maxw = d.dims[i] > maxw ? d.dims[i] : maxw;
  return size_t(2) * 64 * (maxw + 1) * sizeof(float);
}

// Raises the kernel's dynamic-LDS limit (once) so that widths up to
// RDV_MLP_MAX_WIDTH fit; fails if the device has less LDS than needed.
int prepare_chain_f32(const rdv_mlp_desc& d) {
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  const size_t need = chain_lds_bytes(d);
  if (need > di.lds_per_block) return fail(RDV_ERR_UNSUPPORTED, "chain widths need more LDS than the device has");
  static bool raised = false;
  if (!raised) {
    RDV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&mlp_chain_f32_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(di.lds_per_block)));
    raised = true;
  }
  return RDV_OK;
}

// Whether mlp_chain_f32_reg_kernel serves the chain (every width at most 64,
// weights, biases and the activation rows within gfx950's 160 KiB of LDS per
// block), and the LDS bytes it then takes.
constexpr size_t kF32RegLdsCap = 160 * 1024;
bool chain_f32_reg_fits(const rdv_mlp_desc& d, const MlpLayout& lay, size_t* lds_bytes) {
  int64_t floats = 0;
  for (int l = 0; l < d.n_layers; ++l) {
    const int iw = lay.in_w[l], ow = lay.out_w[l];
    if (iw > kF32RegWidth || ow > kF32RegWidth) return false;
    floats += int64_t(ow) * ((iw + 3) & ~3) + ((ow + 3) & ~3);
  }
  const size_t lds = size_t(floats) * 4 + size_t(kF32RegGroups) * 128 * kF32RegActStride * 4;
  if (lds > kF32RegLdsCap) return false;
  if (lds_bytes != nullptr) *lds_bytes = lds;
  return true;
}

// The kernel that evaluates the chain on the vector ALUs for row counts of at
// least kF32RegRows (fewer rows, and the fp32 tail group, take the row kernel).
const char* chain_f32_name(const rdv_mlp_desc& d, const MlpLayout& lay) {
  return chain_f32_reg_fits(d, lay, nullptr) ? "mlp_chain_f32_reg_kernel" : "mlp_chain_f32_kernel";
}

int launch_mlp_chain_f32(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed,
                         const float* x, float* y, int64_t row0, int64_t nrows, bool force_f32,
                         hipStream_t stream, const DirectWeights* dw) {
  if (nrows <= 0) return RDV_OK;
  ChainF32Args a = {};
  a.direct = dw != nullptr ? 1 : 0;
  if (dw != nullptr) a.dw = *dw;
  a.x = x;
  a.y = y;
  a.packed = static_cast<const uint8_t*>(packed);
  a.row0 = row0;
  a.nrows = nrows;
  int maxw = 0;
  for (int i = 0; i <= d.n_layers; ++i) maxw = d.dims[i] > maxw ? d.dims[i] : maxw;
  a.stride = maxw + 1;
  a.force_f32 = force_f32 ? 1 : 0;
  a.encoding = d.encoding;
  a.enc_d = d.in_features;
  a.enc_l = d.enc_octaves;
  for (int i = 0; i < RDV_MLP_MAX_LAYERS; ++i) {
    a.act[i] = i < d.n_layers ? d.act[i] : 0;
    a.prec[i] = i < d.n_layers ? d.prec[i] : 0;
  }
  a.lay = lay;
  size_t reg_lds = 0;
  if (nrows >= kF32RegRows && chain_f32_reg_fits(d, lay, &reg_lds)) {  // the register kernel
    ChainF32RegArgs ra = {};
    int off = 0;
    for (int l = 0; l < d.n_layers; ++l) {
      const int iw = lay.in_w[l], ow = lay.out_w[l];
      ra.in_w[l] = iw;
      ra.out_w[l] = ow;
      ra.act[l] = d.act[l];
      ra.f16[l] = (d.prec[l] == RDV_PREC_F16 && !force_f32) ? 1 : 0;
      ra.wstride[l] = (iw + 3) & ~3;
      ra.woff[l] = off;
      off += ow * ra.wstride[l];
      ra.boff[l] = off;
      off += (ow + 3) & ~3;
    }
    const size_t lds = reg_lds;
    DeviceInfo di;
    int rc = device_info(&di);
    if (rc != RDV_OK) return rc;
    if (lds > di.lds_per_block) return fail(RDV_ERR_UNSUPPORTED, "the fp32 chain needs more LDS than the device has");
    {
      static bool raised = false;
      if (!raised) {
        RDV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&mlp_chain_f32_reg_kernel),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, int(di.lds_per_block)));
        raised = true;
      }
      ra.x = x;
      ra.y = y;
      ra.packed = a.packed;
      ra.row0 = row0;
      ra.nrows = nrows;
      ra.L = d.n_layers;
      ra.encoding = d.encoding;
      ra.enc_d = d.in_features;
      ra.enc_l = d.enc_octaves;
      ra.w_floats = off;
      ra.direct = a.direct;
      ra.dw = a.dw;
      ra.lay = lay;
      int64_t blocks = (nrows + kF32RegRows - 1) / kF32RegRows;
      if (blocks > di.cu_count) blocks = di.cu_count;
      mlp_chain_f32_reg_kernel<<<dim3(unsigned(blocks)), dim3(64 * kF32RegWaves), lds, stream>>>(ra);
      RDV_HIP_TRY(hipGetLastError());
      return RDV_OK;
    }
  }
  const size_t lds = chain_lds_bytes(d);
  const int64_t blocks = (nrows + 63) / 64;
  mlp_chain_f32_kernel<<<dim3(unsigned(blocks)), dim3(64), lds, stream>>>(a);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

}  // namespace rdv
