// Generic chain kernel: one thread per row, every layer on the vector ALUs.
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
  const size_t lds = chain_lds_bytes(d);
  const int64_t blocks = (nrows + 63) / 64;
  mlp_chain_f32_kernel<<<dim3(unsigned(blocks)), dim3(64), lds, stream>>>(a);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

}  // namespace rdv
