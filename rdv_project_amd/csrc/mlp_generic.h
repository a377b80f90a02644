// Runtime-shaped fp16 matrix-core MLP chain: any LinearFast chain of the packed
// layout (mlp_layout.h) -- widths up to 256, up to 16 layers, any per-layer
// activation -- evaluated per 32-point tile with v_mfma_f32_32x32x16_f16, the
// same transposed formulation and D -> B register hand-off as the compile-time
// kernels (mlp_core.h), with the layer shapes read at run time.
//
// MT is the largest number of 32-row M tiles of any layer (1, 2, 4 or 8): it
// sizes the register arrays (MT accumulators, 2 MT hand-off fragments); loops
// run to that bound with wave-uniform guards on the actual layer's shape.
// Layer 0's B fragments are built one K chunk at a time by a caller functor, so
// a wide input (or a long frequency encoding) costs no registers beyond one
// fragment.
//
// Weights are read either from LDS (staged once per block) or straight from
// the packed block in global memory (L2-resident) when the chain's fragments do
// not fit in LDS; each read is one 16-byte access per lane of a 1 KiB fragment.
#ifndef RDV_MLP_GENERIC_H
#define RDV_MLP_GENERIC_H

#include "mlp_core.h"
#include "mlp_layout.h"
#include "rdv_common.h"

namespace rdv {

// Host-computed shape of a chain, passed by value to the kernels.  Fragment
// and bias indices are relative to the first layer's section, so the same
// indices address the LDS copy and the packed block.
struct GenNet {
  int L;                        // layers
  int enc, D, oct;              // input encoding (RDV_ENC_*), raw input width, FREQ octaves
  int out;                      // output width of the last layer
  int mt[RDV_MLP_MAX_LAYERS];   // 32-row M tiles of layer l
  int kc[RDV_MLP_MAX_LAYERS];   // 16-wide K chunks of layer l
  int frag[RDV_MLP_MAX_LAYERS]; // first A fragment (1 KiB units) of layer l
  int bias[RDV_MLP_MAX_LAYERS]; // first bias float of layer l
  int act[RDV_MLP_MAX_LAYERS];  // RDV_ACT_* after layer l
  int f32[RDV_MLP_MAX_LAYERS];  // 1: exact fp32 layer (v_mfma_f32_32x32x2f32, gen_chain_mixed only)
  int kb[RDV_MLP_MAX_LAYERS];   // 32-row K blocks of layer l (fp32 layers)
  int in0;                      // layer 0's input width (the encoded width)
  int n_frag;                   // fragments of the whole chain
  int n_bias;                   // floats spanned by the bias sections (with alignment gaps)
  int max_mt;                   // largest mt[l]
  int64_t frag_off0, bias_off0; // byte offsets of layer 0's sections in the packed block
  int fast;                     // 1: the chain is GenFieldNet with its compact layout (gen_field_row0's compiled path)
};

// The extinction chain the marching kernels carry most often, 3 -> 64 -> 64 ->
// 64 -> 1 with ReLU hidden layers, as a compile-time network: its evaluation
// runs no shape logic (the run-time chain's per-layer switches and loops are
// scalar instructions, and a CU's eight waves share one scalar ALU).
using GenFieldNet = Net<RDV_ENC_NONE, 3, 0, 1, 1, 2, 2, 2, 1>;

// Whether g is network N with N's fragment and bias offsets, fp16 layers and
// ReLU between layers (the head's activation is applied separately).
template <class N>
inline bool gen_matches(const GenNet& g) {
  if (g.L != N::kL || g.enc != N::kEnc || g.D != N::kIn || g.out != N::kOut) return false;
  for (int l = 0; l < N::kL; ++l) {
    if (g.mt[l] != N::mt(l) || g.kc[l] != N::kc(l) || g.frag[l] != N::frag_base(l) || g.bias[l] != N::bias_base(l) ||
        g.f32[l] != 0)
      return false;
    if (l + 1 < N::kL && g.act[l] != RDV_ACT_RELU) return false;
  }
  return true;
}

inline void gen_net(const rdv_mlp_desc& d, const MlpLayout& lay, GenNet* g) {
  g->L = d.n_layers;
  g->enc = d.encoding;
  g->D = d.in_features;
  g->oct = d.enc_octaves;
  g->out = d.dims[d.n_layers];
  g->frag_off0 = lay.frag_off[0];
  g->bias_off0 = lay.bias_off[0];
  g->max_mt = 0;
  for (int l = 0; l < RDV_MLP_MAX_LAYERS; ++l) {
    const bool live = l < d.n_layers;
    g->mt[l] = live ? lay.mt[l] : 0;
    g->kc[l] = live ? lay.kc[l] : 0;
    g->frag[l] = live ? int((lay.frag_off[l] - lay.frag_off[0]) / 1024) : 0;
    g->bias[l] = live ? int((lay.bias_off[l] - lay.bias_off[0]) / 4) : 0;
    g->act[l] = live ? d.act[l] : RDV_ACT_NONE;
    g->f32[l] = live ? lay.f32[l] : 0;
    g->kb[l] = live ? lay.kb[l] : 0;
    if (live && lay.mt[l] > g->max_mt) g->max_mt = lay.mt[l];
  }
  g->in0 = d.dims[0];
  const int last = d.n_layers - 1;
  g->n_frag = int((lay.frag_off[last] - lay.frag_off[0]) / 1024) + lay.frag_units[last];
  g->n_bias = int((lay.bias_off[last] - lay.bias_off[0]) / 4) + 32 * lay.mt[last];
  g->fast = gen_matches<GenFieldNet>(*g) ? 1 : 0;
}

// Waves per block of the kernels built on gen_chain: 8 per CU (2 per SIMD);
// the 8-tile chains (widths up to 256) use 4 (one per SIMD), whose 512
// registers hold their 8 accumulators.
template <int MT>
constexpr int gen_waves() { return MT >= 8 ? 4 : 8; }

// Bytes of LDS a block needs to hold the chain's fragments and biases.
inline int64_t gen_lds_bytes(const GenNet& g) { return int64_t(g.n_frag) * 1024 + int64_t(g.n_bias) * 4; }

// Register-array bound for a chain: the smallest of 1, 2, 4, 8 covering max_mt.
inline int gen_mt_bound(const GenNet& g) {
  int m = 1;
  while (m < g.max_mt) m *= 2;
  return m;
}

// Copies the fragments and biases into LDS: fragments at byte 0, biases after.
__device__ __forceinline__ void gen_stage(const uint8_t* packed, const GenNet& g, uint8_t* smem) {
  const uint4* fs = reinterpret_cast<const uint4*>(packed + g.frag_off0);
  uint4* fd = reinterpret_cast<uint4*>(smem);
  const int nf = g.n_frag * 64;  // 16-byte units
  for (int i = threadIdx.x; i < nf; i += blockDim.x) fd[i] = fs[i];
  const float* bsrc = reinterpret_cast<const float*>(packed + g.bias_off0);
  float* bd = reinterpret_cast<float*>(smem + int64_t(g.n_frag) * 1024);
  for (int i = threadIdx.x; i < g.n_bias; i += blockDim.x) bd[i] = bsrc[i];
}

// Output feature of D register j (0..15) of M tile t for lane half h.
__device__ __forceinline__ int gen_row(int t, int j, int h) { return 32 * t + 8 * (j >> 2) + 4 * h + (j & 3); }

// Head activation of the last layer at run time (transcendental heads on the
// hardware exp2 / log2 / rcp, as in the compile-time kernels).
__device__ __forceinline__ float gen_head_act(int act, int channel, float v) {
  switch (act) {
    case RDV_ACT_RELU: return fmaxf(v, 0.0f);
    case RDV_ACT_SOFTPLUS: return fast_softplus(v);
    case RDV_ACT_SIGMOID: return fast_sigmoid(v);
    case RDV_ACT_DENSITY_RGB: return channel == 0 ? fast_softplus(v) : fast_sigmoid(v);
    default: return v;
  }
}

// D registers of an M-tile layer -> B fragments 0 .. 2M - 1 of the next layer,
// after activation ACT (ReLU after the fp16 rounding, which is monotone, so
// the same value; the transcendental activations in fp32 before it, on the
// hardware exp2 / log2 / rcp like the heads).  ACT < 0: `act` read per value.
template <int MT, int M, int ACT>
__device__ __forceinline__ void gen_handoff_t(const f32x16 (&acc)[M], half8 (&b)[2 * MT], int act, int h) {
  const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int t = 0; t < M; ++t) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      half8 v;
      if constexpr (ACT == RDV_ACT_RELU || ACT == RDV_ACT_NONE) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = half_t(acc[t][8 * q + j]);
        if constexpr (ACT == RDV_ACT_RELU) v = __builtin_elementwise_max(v, zero);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = half_t(gen_head_act(act, gen_row(t, 8 * q + j, h), acc[t][8 * q + j]));
      }
      b[2 * t + q] = v;
    }
  }
}

template <int MT, int M>
__device__ __forceinline__ void gen_handoff(const f32x16 (&acc)[M], half8 (&b)[2 * MT], int act, int h) {
  if (act == RDV_ACT_RELU) gen_handoff_t<MT, M, RDV_ACT_RELU>(acc, b, act, h);
  else if (act == RDV_ACT_NONE) gen_handoff_t<MT, M, RDV_ACT_NONE>(acc, b, act, h);
  else gen_handoff_t<MT, M, -1>(acc, b, act, h);
}

// Accumulators of an M-tile layer start at its bias (or zero): rows 32t + 8q + 4h + 0..3.
template <int M>
__device__ __forceinline__ void gen_init(f32x16 (&acc)[M], const float* bias, bool has_bias, int h) {
#pragma unroll
  for (int t = 0; t < M; ++t) {
    if (has_bias) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 bv = *reinterpret_cast<const f32x4*>(bias + 32 * t + 8 * q + 4 * h);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[t][4 * q + jj] = bv[jj];
      }
    } else {
      acc[t] = f32x16{};
    }
  }
}

// Shape of one hidden or last layer, read once at the layer's start.
struct GenLayerShape {
  int kc, frag, bias, act;  // as GenNet's entries of the layer
  bool last;                // the chain's last layer
};

// Per-layer context of gen_chain.
struct GenCtx {
  const float* bias;  // the chain's biases (LDS or global)
  bool has_bias;
  int h;
};

// The layer's accumulators go to the next layer's fragments, or, for the last
// layer, to sink(acc) (acc: f32x16[M], before the head activation).
template <int MT, int M, class Sink>
__device__ __forceinline__ void gen_finish(const f32x16 (&acc)[M], half8 (&b)[2 * MT], bool last, int act, int h,
                                           Sink&& sink) {
  if (last) sink(acc);
  else gen_handoff<MT, M>(acc, b, act, h);
}

// No-op hook of gen_chain.
struct GenNoHook {
  __device__ __forceinline__ void operator()() const {}
};

// Layer 0 with M tiles, B fragment of K chunk c from l0(c).  KC0 == 0: a
// run-time loop over the chunks, one at a time.  KC0 > 0 (the chain has at most
// KC0 chunks in layer 0): the loop is unrolled, so l0 may index registers by c,
// and the A fragments are double-buffered as in gen_layer.  after0() runs after
// the layer's MFMAs are issued, before its hand-off.
template <int MT, int M, int KC0, class W, class L0, class Sink, class Hook>
__device__ __forceinline__ void gen_layer0(const GenNet& g, const GenCtx& x, const W& wf, L0&& l0, half8 (&b)[2 * MT],
                                           Sink&& sink, Hook&& after0) {
  f32x16 acc[M];
  gen_init<M>(acc, x.bias + g.bias[0], x.has_bias, x.h);
  const int kc = g.kc[0], f0 = g.frag[0];
  if constexpr (KC0 == 0) {
    for (int c = 0; c < kc; ++c) {
      half8 A[M];
#pragma unroll
      for (int t = 0; t < M; ++t) A[t] = wf(f0 + t * kc + c);
      const half8 bc = l0(c);
#pragma unroll
      for (int t = 0; t < M; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[t], bc, acc[t], 0, 0, 0);
    }
  } else {
    half8 A[2][M];
#pragma unroll
    for (int t = 0; t < M; ++t) A[0][t] = wf(f0 + t * kc);
#pragma unroll
    for (int c = 0; c < KC0; ++c) {
      if (c < kc) {
        const int cn = c + 1 < kc ? c + 1 : c;
#pragma unroll
        for (int t = 0; t < M; ++t) A[(c + 1) & 1][t] = wf(f0 + t * kc + cn);
        const half8 bc = l0(c);
#pragma unroll
        for (int t = 0; t < M; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[c & 1][t], bc, acc[t], 0, 0, 0);
      }
    }
  }
  after0();
  gen_finish<MT, M>(acc, b, g.L == 1, g.act[0], x.h, sink);
}

// K chunks of A fragments a layer with M tiles keeps in flight: eight
// fragments (32 VGPRs) for every M up to 4, so a narrow layer, whose few MFMAs
// per chunk cannot cover one LDS read latency, reads several chunks ahead.
template <int M>
constexpr int gen_ring() { return M == 1 ? 8 : M == 2 ? 4 : 2; }

// Hidden or last layer l with M tiles and kc = 2 mt[l - 1] K chunks from b: A
// fragments in a register ring of R = gen_ring<M>() chunks, chunk c + R - 1's
// reads issued before chunk c's MFMAs.  Reads past the last chunk re-read it
// (a valid fragment, no branch), so every path issues the same reads.
template <int MT, int M, class W, class Sink>
__device__ __forceinline__ void gen_layer(const GenLayerShape& s, const GenCtx& x, const W& wf, half8 (&b)[2 * MT],
                                          Sink&& sink) {
  constexpr int R = gen_ring<M>() < 2 * MT ? gen_ring<M>() : 2 * MT;
  f32x16 acc[M];
  gen_init<M>(acc, x.bias + s.bias, x.has_bias, x.h);
  const int kc = s.kc, f0 = s.frag;
  half8 A[R][M];
#pragma unroll
  for (int p = 0; p + 1 < R; ++p) {
    const int cp = p < kc ? p : kc - 1;
#pragma unroll
    for (int t = 0; t < M; ++t) A[p][t] = wf(f0 + t * kc + cp);
  }
#pragma unroll
  for (int c = 0; c < 2 * MT; ++c) {
    if (c < kc) {
      const int cn = c + R - 1 < kc ? c + R - 1 : kc - 1;
#pragma unroll
      for (int t = 0; t < M; ++t) A[(c + R - 1) % R][t] = wf(f0 + t * kc + cn);
#pragma unroll
      for (int t = 0; t < M; ++t)
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[c % R][t], b[c], acc[t], 0, 0, 0);
    }
  }
  gen_finish<MT, M>(acc, b, s.last, s.act, x.h, sink);
}

#define RDV_GEN_SWITCH(mt, CALL)                                     \
  switch (mt) {                                                      \
    case 1: CALL(1); break;                                          \
    case 2: if constexpr (MT >= 2) { CALL(2); } break;               \
    case 3: if constexpr (MT >= 3) { CALL(3); } break;               \
    case 4: if constexpr (MT >= 4) { CALL(4); } break;               \
    case 5: if constexpr (MT >= 5) { CALL(5); } break;               \
    case 6: if constexpr (MT >= 6) { CALL(6); } break;               \
    case 7: if constexpr (MT >= 7) { CALL(7); } break;               \
    default: if constexpr (MT >= 8) { CALL(8); } break;              \
  }

// The whole chain for one 32-point tile.  l0(c) returns this lane's B fragment
// of layer 0's K chunk c; wf(f) returns A fragment f (this lane's 16 bytes).
// The last layer's accumulators (f32x16[mt], before its activation) go to
// sink(acc); the register arrays between layers are only the 2 MT fragments.
// KC0 and after0: as in gen_layer0.
template <int MT, int KC0 = 0, class W, class L0, class Sink, class Hook = GenNoHook>
__device__ __forceinline__ void gen_chain(const GenNet& g, const GenCtx& x, const W& wf, L0&& l0, Sink&& sink,
                                          Hook&& after0 = Hook{}) {
  half8 b[2 * MT];
#define RDV_GEN_L0(M) gen_layer0<MT, M, KC0>(g, x, wf, l0, b, sink, after0)
  RDV_GEN_SWITCH(g.mt[0], RDV_GEN_L0)
#undef RDV_GEN_L0
#pragma nounroll
  for (int l = 1; l < g.L; ++l) {
    const GenLayerShape s{g.kc[l], g.frag[l], g.bias[l], g.act[l], l == g.L - 1};
    const int mt = g.mt[l];
    // The layer's shape is in SGPRs before its first LDS read: the wait for
    // these scalar loads would otherwise also wait for the bias reads.
    asm volatile("" ::"s"(s.kc), "s"(s.frag), "s"(s.bias), "s"(s.act), "s"(mt));
#define RDV_GEN_LH(M) gen_layer<MT, M>(s, x, wf, b, sink)
    RDV_GEN_SWITCH(mt, RDV_GEN_LH)
#undef RDV_GEN_LH
  }
}

// Feature f of a FREQ encoding of the point p[0..D) (get(d) returns p[d]):
// f < D: p_f; then per octave k the D sines sin(2^k pi p_d) and the D cosines.
// v_sin / v_cos take revolutions: 2^k pi p = 2 pi (2^(k-1) p), and the power of
// two scaling and the fractional part are exact, so the argument is reduced
// without error before the hardware evaluates it.
template <class Get>
__device__ __forceinline__ float gen_freq_feature(int f, int D, Get&& get) {
  if (f < 0) return 0.0f;
  if (f < D) return get(f);
  const int k = (f - D) / (2 * D), r = (f - D) % (2 * D);
  const bool is_cos = r >= D;
  const float rev = __builtin_amdgcn_fractf(__builtin_ldexpf(get(is_cos ? r - D : r), k - 1));
  return is_cos ? __builtin_amdgcn_cosf(rev) : __builtin_amdgcn_sinf(rev);
}

// Layer-0 B fragment of K chunk c for a point whose raw coordinates are read by
// get(d), d < D: raw slots (identity) or the FREQ slot order of mlp_layout.h.
template <class Get>
__device__ __forceinline__ half8 gen_l0_chunk(const GenNet& g, int c, int h, Get&& get) {
  half8 b;
  if (g.enc == RDV_ENC_FREQ) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      b[j] = half_t(gen_freq_feature(layer0_slot_feature(RDV_ENC_FREQ, g.D, g.oct, 16 * c + 8 * h + j), g.D, get));
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int f = 16 * c + 8 * h + j;
      b[j] = half_t(f < g.D ? get(f) : 0.0f);
    }
  }
  return b;
}


// ----------------------------------------------------------- mixed chains
// Chains with exact fp32 layers (Linear, maps/linear.h) alone or mixed with
// LinearFast layers, on the matrix cores: an fp32 layer runs
// v_mfma_f32_32x32x2f32 with its fp32 fragments (mlp_layout.h), one MFMA per
// input row pair, B = the producing layer's fp32 D register after its
// activation (no fp16 rounding anywhere in an fp32 layer, as in the
// reference's Linear); an fp16 layer is the LinearFast layer of gen_chain,
// and its input is rounded to fp16 by the hand-off whatever produced it.  The
// fp32 products and sums are the matrix core's fp32 arithmetic, in its own
// order (the reference sums one input at a time).
//
// MT bounds every layer's M tiles (register arrays: MT fp32 input blocks and
// 2 MT fp16 fragments between layers).  feat(k) returns this lane's value of
// encoded input feature k (0 past the input width).

// fp32 layer with M tiles over the kb input blocks in v (hidden layer) or from
// feat (layer 0, kb input blocks of its width); accumulates into acc.
template <int MT, int M, bool L0, class W, class Feat>
__device__ __forceinline__ void gen_f32_layer(f32x16 (&acc)[M], int f0, int kb, int width, int h, const W& wf,
                                              Feat& feat, const f32x16 (&v)[MT]) {
  if constexpr (L0) {
    for (int blk = 0; blk < kb; ++blk) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 A[M];
#pragma unroll
        for (int t = 0; t < M; ++t) A[t] = __builtin_bit_cast(f32x4, wf(f0 + (t * kb + blk) * 4 + q));
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int k0 = 32 * blk + 8 * q + jj;  // lane half 0's row; half 1 reads k0 + 4
          if (k0 < width) {
            const float bv = feat(k0 + 4 * h);
#pragma unroll
            for (int t = 0; t < M; ++t) {
              const float av = A[t][jj];
              acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc[t], 0, 0, 0);
            }
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int blk = 0; blk < MT; ++blk) {
      if (blk < kb) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f32x4 A[M];
#pragma unroll
          for (int t = 0; t < M; ++t) A[t] = __builtin_bit_cast(f32x4, wf(f0 + (t * kb + blk) * 4 + q));
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const float bv = v[blk][4 * q + jj];
#pragma unroll
            for (int t = 0; t < M; ++t) {
              const float av = A[t][jj];
              acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc[t], 0, 0, 0);
            }
          }
        }
      }
    }
  }
}

// One layer l of a mixed chain with M tiles.
template <int MT, int M, class W, class Feat, class Get, class Sink>
__device__ __forceinline__ void gen_mixed_layer(const GenNet& g, int l, const GenCtx& x, const W& wf, Feat& feat,
                                                Get& get, half8 (&b)[2 * MT], f32x16 (&v)[MT], Sink& sink) {
  f32x16 acc[M];
  gen_init<M>(acc, x.bias + g.bias[l], x.has_bias, x.h);
  const int f0 = g.frag[l];
  if (g.f32[l]) {
    if (l == 0) gen_f32_layer<MT, M, true>(acc, f0, g.kb[0], g.in0, x.h, wf, feat, v);
    else gen_f32_layer<MT, M, false>(acc, f0, g.kb[l], 0, x.h, wf, feat, v);
  } else if (l == 0) {
    const int kc = g.kc[0];
    for (int c = 0; c < kc; ++c) {
      const half8 bc = gen_l0_chunk(g, c, x.h, get);
#pragma unroll
      for (int t = 0; t < M; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf(f0 + t * kc + c), bc, acc[t], 0, 0, 0);
    }
  } else {
    const int kc = g.kc[l];
#pragma unroll
    for (int c = 0; c < 2 * MT; ++c) {
      if (c < kc) {
#pragma unroll
        for (int t = 0; t < M; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf(f0 + t * kc + c), b[c], acc[t], 0, 0, 0);
      }
    }
  }
  const bool last = l == g.L - 1;
  if (last) {
    sink(acc);
  } else if (g.f32[l + 1]) {  // the next layer reads fp32 rows: the activation in fp32, no rounding
#pragma unroll
    for (int t = 0; t < M; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) v[t][j] = gen_head_act(g.act[l], gen_row(t, j, x.h), acc[t][j]);
  } else {
    gen_handoff<MT, M>(acc, b, g.act[l], x.h);
  }
}

// The whole mixed chain for one 32-point tile: get(d) returns raw coordinate d
// of this lane's point; sink(acc) receives the last layer's accumulators.
template <int MT, class W, class Get, class Sink>
__device__ __forceinline__ void gen_chain_mixed(const GenNet& g, const GenCtx& x, const W& wf, Get&& get, Sink&& sink) {
  half8 b[2 * MT];
  f32x16 v[MT];
  const int enc_w = g.enc == RDV_ENC_FREQ ? g.D * (1 + 2 * g.oct) : g.D;
  auto feat = [&](int k) -> float {
    if (k >= enc_w) return 0.0f;
    if (g.enc == RDV_ENC_FREQ) return gen_freq_feature(k, g.D, get);
    return get(k);
  };
#pragma nounroll
  for (int l = 0; l < g.L; ++l) {
#define RDV_GEN_LM(M) gen_mixed_layer<MT, M>(g, l, x, wf, feat, get, b, v, sink)
    RDV_GEN_SWITCH(g.mt[l], RDV_GEN_LM)
#undef RDV_GEN_LM
  }
}

}  // namespace rdv

#endif  // RDV_MLP_GENERIC_H
