// Packs fp32 nn.Linear-layout weights into the layout of mlp_layout.h.
#include "mlp_layout.h"
#include "rdv_common.h"

namespace rdv {

__global__ void mlp_pack_header_kernel(uint8_t* __restrict__ packed) {
  if (threadIdx.x == 0) {
    MlpPackHeader* hdr = reinterpret_cast<MlpPackHeader*>(packed);
    hdr->magic = kMlpPackMagic;
    hdr->flags = 0;
  }
}

// One thread per element of the largest region of layer `li`.
__global__ void mlp_pack_layer_kernel(const float* __restrict__ W, const float* __restrict__ b,
                                      uint8_t* __restrict__ packed, MlpLayout lay, int li,
                                      int encoding, int enc_d, int enc_l) {
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
  }
  // fp16 A fragments: element e = ((t * kc + c) * 64 + lane) * 8 + j
  const int64_t n_frag = lay.f32[li] ? 0 : int64_t(mt) * kc * 64 * 8;
  if (e < n_frag) {
    const int j = int(e & 7);
    const int lane = int((e >> 3) & 63);
    const int64_t tc = e >> 9;
    const int c = int(tc % kc), t = int(tc / kc);
    const int m = 32 * t + (lane & 31);
    const int kv = 16 * c + 8 * (lane >> 5) + j;
    const int ka = li == 0 ? layer0_slot_feature(encoding, enc_d, enc_l, kv) : hidden_slot_feature(kv);
    float v = 0.0f;
    if (m < out_w && ka >= 0 && ka < in_w) v = W[int64_t(m) * in_w + ka];
    reinterpret_cast<half_t*>(packed + lay.frag_off[li])[e] = half_t(v);
  }
  // padded fp32 bias
  if (e < int64_t(mt) * 32) {
    const float bv = e < out_w ? b[e] : 0.0f;
    reinterpret_cast<float*>(packed + lay.bias_off[li])[e] = bv;
    if (bv != 0.0f) atomicOr(&reinterpret_cast<MlpPackHeader*>(packed)->flags, kMlpHasBias);
  }
  // fp32 copies
  if (e < int64_t(out_w) * in_w) reinterpret_cast<float*>(packed + lay.w32_off[li])[e] = W[e];
  if (e < out_w) reinterpret_cast<float*>(packed + lay.b32_off[li])[e] = b[e];
}

int launch_mlp_pack(const rdv_mlp_desc& d, const MlpLayout& lay, const float* const* W,
                    const float* const* b, void* packed, hipStream_t stream) {
  mlp_pack_header_kernel<<<1, 64, 0, stream>>>(static_cast<uint8_t*>(packed));
  RDV_HIP_TRY(hipGetLastError());
  for (int i = 0; i < lay.n_layers; ++i) {
    int64_t n = int64_t(lay.frag_units[i]) * 256;  // fragment elements (512 fp16 or 256 fp32 per KiB) bound
    if (!lay.f32[i]) n = int64_t(lay.mt[i]) * lay.kc[i] * 64 * 8;
    const int64_t nw = int64_t(lay.out_w[i]) * lay.in_w[i];
    if (nw > n) n = nw;
    const int threads = 256;
    const int64_t blocks = (n + threads - 1) / threads;
    mlp_pack_layer_kernel<<<dim3(unsigned(blocks)), dim3(threads), 0, stream>>>(
        W[i], b[i], static_cast<uint8_t*>(packed), lay, i, d.encoding, d.in_features, d.enc_octaves);
    RDV_HIP_TRY(hipGetLastError());
  }
  return RDV_OK;
}

}  // namespace rdv
