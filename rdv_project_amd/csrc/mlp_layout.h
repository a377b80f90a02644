// Packed parameter block of a fused MLP, shared by the packer and every MLP kernel.
//
// Matrix-core formulation.  Each layer is evaluated transposed, H^T = W . X^T,
// with v_mfma_f32_32x32x16_f16: A = a 32x16 tile of W (output features x input
// features), B = a 16x32 tile of X^T (input features x 32 points), D = 32 output
// features x 32 points in fp32.  Per lane l (h = l / 32):
//   A operand: W[32t + l%32][virtual k = 16c + 8h + j], j = 0..7
//   B operand: X^T[virtual k = 16c + 8h + j][point l%32]
//   D result : row 32t + 8(j/4) + 4h + (j%4) of point l%32, j = 0..15
// The D registers of one 32-row tile, converted to fp16, ARE the B operands of
// the next layer's two 16-wide K chunks (registers 0..7 -> chunk 2t, 8..15 ->
// chunk 2t+1), with virtual k = 16c + v holding actual feature
// 16c + sigma(v), where sigma swaps the middle two quartets of a 16-chunk.
// The next layer's weight columns are permuted by the same sigma when packed,
// so activations never leave registers between layers.
//
// Exact fp32 layers (RDV_PREC_F32) on the matrix cores use
// v_mfma_f32_32x32x2f32 in the same transposed formulation: A = W[32t + l%32]
// [k], B = the input row k of point l%32, one fp32 value per lane, K = 2 (lane
// half h supplies k = the half's row).  MFMA j (0..15) of 32-row input block kb
// takes k = 32kb + 8(j/4) + 4h + (j%4), which is exactly the row that D
// register j of the producing layer holds: a layer's fp32 D registers (after
// its activation) ARE the next fp32 layer's B operands, one per MFMA, with no
// permutation.  The A values of MFMAs 4q .. 4q+3 for lane l are the four
// consecutive columns W[m][32kb + 8q + 4h + 0..3], one 16-byte read.  Layer 0
// reads its input rows in the same order (feature k = the encoded feature k).
//
// Layout (every section 256-byte aligned), for layer i with KC = K chunks of 16,
// KB = K blocks of 32 and MT = M tiles of 32:
//   header  : MlpPackHeader, 256 bytes (flags computed by the packer)
//   frag[i] : fp16 layer: MT x KC x 64 lanes x 8 fp16 (A fragments in lane order)
//             fp32 layer: MT x KB x 4 quartets x 64 lanes x 4 fp32
//   bias[i] : MT*32 fp32                      (zero padded)
//   w32[i]  : dims[i+1] x dims[i] fp32        (row-major copy, for fp32 paths)
//   b32[i]  : dims[i+1] fp32
// Both fragment kinds come in 1 KiB units (frag_units[i] of them).
#pragma once

#include <stdint.h>

#include "../../include/rdv_hip.h"

namespace rdv {

// First 256 bytes of a packed block.
// Each word is written by exactly one thread of the single pack launch, so no
// word needs clearing first: layer_bias[i] by the block that packs layer i's
// bias, the rest by layer 0's.
struct MlpPackHeader {
  uint32_t magic;                             // kMlpPackMagic once packed
  uint32_t reserved;
  uint32_t layer_bias[RDV_MLP_MAX_LAYERS];  // 1: layer i has a non-zero bias element (0 past the last layer)
};
constexpr uint32_t kMlpPackMagic = 0x52445632u;  // "RDV2"

// Whether any layer of a packed block has a non-zero bias (the kernels then
// seed their accumulators with the biases; otherwise MFMA's zero C operand).
__host__ __device__ inline bool packed_has_bias(const uint8_t* packed) {
  const MlpPackHeader* h = reinterpret_cast<const MlpPackHeader*>(packed);
  uint32_t any = 0;
#pragma unroll
  for (int i = 0; i < RDV_MLP_MAX_LAYERS; ++i) any |= h->layer_bias[i];
  return any != 0;
}
constexpr int64_t kMlpHeaderBytes = 256;

struct MlpLayout {
  int n_layers;
  int in_w[RDV_MLP_MAX_LAYERS];   // actual input width of layer i
  int out_w[RDV_MLP_MAX_LAYERS];  // actual output width of layer i
  int kc[RDV_MLP_MAX_LAYERS];     // K chunks of 16 (virtual, after slot mapping)
  int kb[RDV_MLP_MAX_LAYERS];     // K blocks of 32 (fp32 layers' matrix-core path)
  int mt[RDV_MLP_MAX_LAYERS];     // M tiles of 32
  int f32[RDV_MLP_MAX_LAYERS];    // 1: exact fp32 layer (fp32 fragments)
  int frag_units[RDV_MLP_MAX_LAYERS];  // 1 KiB units of layer i's fragments
  int64_t frag_off[RDV_MLP_MAX_LAYERS];
  int64_t bias_off[RDV_MLP_MAX_LAYERS];
  int64_t w32_off[RDV_MLP_MAX_LAYERS];
  int64_t b32_off[RDV_MLP_MAX_LAYERS];
  int64_t total_bytes;
};

// The layers' own parameters for the kernels that read them without a packed
// block: W[i] row-major fp32 [dims[i+1], dims[i]] (nn.Linear layout), b[i] fp32
// [dims[i+1]], device pointers.
struct DirectWeights {
  const float* W[RDV_MLP_MAX_LAYERS];
  const float* b[RDV_MLP_MAX_LAYERS];
};

__host__ __device__ inline int div_up(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ inline int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

// Octaves of a FREQ encoding evaluated by lane half 0 (the rest go to half 1).
__host__ __device__ inline int freq_octaves_half0(int L) { return (L + 1) / 2; }

// K chunks layer 0 needs on the matrix-core path.
__host__ __device__ inline int layer0_kc(int encoding, int D, int L, int enc_width) {
  if (encoding == RDV_ENC_FREQ) {
    int h0 = freq_octaves_half0(L);
    int need0 = 2 * D * h0 + D;  // half 0: trig slots of its octaves, then the raw input
    int need1 = 2 * D * (L - h0);
    int need = need0 > need1 ? need0 : need1;
    return div_up(need, 8);
  }
  return div_up(enc_width, 16);
}

// Actual feature index (column of layer 0's weight) that virtual K slot kv of
// layer 0 carries, or -1 for a zero slot.
//  NONE: identity.
//  FREQ: within each lane half, slot s = 8c + j holds, for the half's octaves
//        k (half 0: [0, h0), half 1: [h0, L)), in order: sin(2^k pi p_d) for
//        d < D, then cos(2^k pi p_d); half 0 then holds p_d itself.  Both halves
//        therefore evaluate the same function kind in the same slot.
__host__ __device__ inline int layer0_slot_feature(int encoding, int D, int L, int kv) {
  if (encoding != RDV_ENC_FREQ) return kv;
  const int c = kv >> 4, h = (kv >> 3) & 1, j = kv & 7;
  const int s = c * 8 + j;
  const int h0 = freq_octaves_half0(L);
  const int nh = h == 0 ? h0 : L - h0;
  const int kbase = h == 0 ? 0 : h0;
  if (s < 2 * D * nh) {
    const int i = s / (2 * D), r = s % (2 * D);
    const int k = kbase + i;
    const bool is_cos = r >= D;
    const int d = is_cos ? r - D : r;
    return D + 2 * D * k + (is_cos ? D : 0) + d;
  }
  if (h == 0 && s >= 2 * D * h0 && s < 2 * D * h0 + D) return s - 2 * D * h0;
  return -1;
}

// sigma: swaps quartets 1 and 2 of a 16-chunk (self-inverse).
__host__ __device__ inline int chunk_sigma(int v) {
  const int q = v >> 2;
  const int q2 = (q == 1) ? 2 : (q == 2 ? 1 : q);
  return (q2 << 2) | (v & 3);
}

// Feature of layer i >= 1 carried by virtual K slot kv.
__host__ __device__ inline int hidden_slot_feature(int kv) { return (kv & ~15) | chunk_sigma(kv & 15); }

// Fills `lay` from `d`; returns false if d is not a valid chain.
inline bool mlp_layout(const rdv_mlp_desc& d, MlpLayout* lay) {
  const int L = d.n_layers;
  if (L < 1 || L > RDV_MLP_MAX_LAYERS) return false;
  lay->n_layers = L;
  int64_t off = kMlpHeaderBytes;
  for (int i = 0; i < L; ++i) {
    lay->in_w[i] = d.dims[i];
    lay->out_w[i] = d.dims[i + 1];
    lay->mt[i] = div_up(d.dims[i + 1], 32);
    lay->kc[i] = i == 0 ? layer0_kc(d.encoding, d.in_features, d.enc_octaves, d.dims[0])
                        : 2 * lay->mt[i - 1];
    lay->kb[i] = i == 0 ? div_up(d.dims[0], 32) : lay->mt[i - 1];
    lay->f32[i] = d.prec[i] == RDV_PREC_F32 ? 1 : 0;
    lay->frag_units[i] = lay->f32[i] ? lay->mt[i] * lay->kb[i] * 4 : lay->mt[i] * lay->kc[i];
  }
  for (int i = 0; i < L; ++i) {
    lay->frag_off[i] = off;
    off = align256(off + int64_t(lay->frag_units[i]) * 1024);
  }
  for (int i = 0; i < L; ++i) {
    lay->bias_off[i] = off;
    off = align256(off + int64_t(lay->mt[i]) * 32 * 4);
  }
  for (int i = 0; i < L; ++i) {
    lay->w32_off[i] = off;
    off = align256(off + int64_t(lay->out_w[i]) * lay->in_w[i] * 4);
  }
  for (int i = 0; i < L; ++i) {
    lay->b32_off[i] = off;
    off = align256(off + int64_t(lay->out_w[i]) * 4);
  }
  lay->total_bytes = off;
  return true;
}

}  // namespace rdv
