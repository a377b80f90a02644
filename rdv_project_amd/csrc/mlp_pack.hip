// Packs fp32 nn.Linear-layout weights into the layout of mlp_layout.h, every
// layer and the header in one launch (grid.y = layer).
#include "mlp_layout.h"
#include "rdv_common.h"

namespace rdv {

struct PackArgs {
  DirectWeights dw;
  MlpLayout lay;
  int encoding, enc_d, enc_l;
};

constexpr int kPackThreads = 256;  // >= the widest padded bias (8 M tiles of 32)

// One thread per element of the largest region of layer blockIdx.y.
__global__ __launch_bounds__(kPackThreads) void mlp_pack_kernel(PackArgs a, uint8_t* __restrict__ packed) {
  const int li = int(blockIdx.y);
  const MlpLayout& lay = a.lay;
  const float* __restrict__ W = a.dw.W[li];
  const float* __restrict__ b = a.dw.b[li];
  const int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int in_w = lay.in_w[li], out_w = lay.out_w[li];
  const int kc = lay.kc[li], mt = lay.mt[li];

  if (lay.f32[li]) {
    // fp32 A fragments: element e = (((t * kb + blk) * 4 + q) * 64 + lane) * 4 + jj
    // holds W[32t + lane % 32][32 blk + 8q + 4 (lane / 32) + jj]
    const int kb = lay.kb[li];
    if (e < int64_t(mt) * kb * 4 * 64 * 4) {
      const int jj = int(e & 3);
      const int lane = int((e >> 2) & 63);
      const int64_t grp = e >> 8;
      const int q = int(grp & 3);
      const int64_t tb = grp >> 2;
      const int blk = int(tb % kb), t = int(tb / kb);
      const int m = 32 * t + (lane & 31);
      const int k = 32 * blk + 8 * q + 4 * (lane >> 5) + jj;
      const float v = (m < out_w && k < in_w) ? W[int64_t(m) * in_w + k] : 0.0f;
      reinterpret_cast<float*>(packed + lay.frag_off[li])[e] = v;
    }
  } else if (e < int64_t(mt) * kc * 64 * 8) {
    // fp16 A fragments: element e = ((t * kc + c) * 64 + lane) * 8 + j
    const int j = int(e & 7);
    const int lane = int((e >> 3) & 63);
    const int64_t tc = e >> 9;
    const int c = int(tc % kc), t = int(tc / kc);
    const int m = 32 * t + (lane & 31);
    const int kv = 16 * c + 8 * (lane >> 5) + j;
    const int ka = li == 0 ? layer0_slot_feature(a.encoding, a.enc_d, a.enc_l, kv) : hidden_slot_feature(kv);
    float v = 0.0f;
    if (m < out_w && ka >= 0 && ka < in_w) v = W[int64_t(m) * in_w + ka];
    reinterpret_cast<half_t*>(packed + lay.frag_off[li])[e] = half_t(v);
  }
  // padded fp32 bias
  if (e < int64_t(mt) * 32) {
    const float bv = e < out_w ? b[e] : 0.0f;
    reinterpret_cast<float*>(packed + lay.bias_off[li])[e] = bv;
  }
  // fp32 copies
  if (e < int64_t(out_w) * in_w) reinterpret_cast<float*>(packed + lay.w32_off[li])[e] = W[e];
  if (e < out_w) reinterpret_cast<float*>(packed + lay.b32_off[li])[e] = b[e];
  // header: block 0 of each layer covers its whole bias (mt * 32 <= kPackThreads)
  if (blockIdx.x == 0) {
    const bool nz = int(threadIdx.x) < out_w && b[threadIdx.x < unsigned(out_w) ? threadIdx.x : 0] != 0.0f;
    const int any = __syncthreads_or(nz ? 1 : 0);
    MlpPackHeader* hdr = reinterpret_cast<MlpPackHeader*>(packed);
    if (threadIdx.x == 0) hdr->layer_bias[li] = any ? 1u : 0u;
    if (li == 0) {
      if (threadIdx.x == 0) {
        hdr->magic = kMlpPackMagic;
        hdr->reserved = 0;
      }
      if (int(threadIdx.x) >= lay.n_layers && threadIdx.x < RDV_MLP_MAX_LAYERS) hdr->layer_bias[threadIdx.x] = 0;
    }
  }
}

int launch_mlp_pack(const rdv_mlp_desc& d, const MlpLayout& lay, const float* const* W, const float* const* b,
                    void* packed, hipStream_t stream) {
  PackArgs a = {};
  int64_t n = kPackThreads;
  for (int i = 0; i < lay.n_layers; ++i) {
    a.dw.W[i] = W[i];
    a.dw.b[i] = b[i];
    int64_t ni = lay.f32[i] ? int64_t(lay.frag_units[i]) * 256 : int64_t(lay.mt[i]) * lay.kc[i] * 64 * 8;
    const int64_t nw = int64_t(lay.out_w[i]) * lay.in_w[i];
    if (nw > ni) ni = nw;
    if (ni > n) n = ni;
  }
  a.lay = lay;
  a.encoding = d.encoding;
  a.enc_d = d.in_features;
  a.enc_l = d.enc_octaves;
  const int64_t blocks = (n + kPackThreads - 1) / kPackThreads;
  mlp_pack_kernel<<<dim3(unsigned(blocks), unsigned(lay.n_layers)), dim3(kPackThreads), 0, stream>>>(
      a, static_cast<uint8_t*>(packed));
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

}  // namespace rdv
