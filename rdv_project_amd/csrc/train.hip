// MLP training step on the matrix cores: forward, MSE loss, backward with fp32
// weight gradients reduced over every point (build-defined; the reference has
// no backward pass).
//
// Numerics.  Forward = the LinearFast chain (fp16 inputs and weights, fp32
// accumulation, fp32 bias, ReLU); hidden activations are kept in fp16 exactly
// as they feed the next layer.  Loss = mean over n x out of (y - t)^2.  The
// backward carries the unscaled gradient g = 2 (y - t) (fp16, O(1) values, no
// underflow); dz_l = (dz_{l+1} W_l) masked by h_l > 0 in fp32, rounded to fp16;
// dW_l = sum_p dz_{l+1}[p]^T h_l[p] and db_l = sum_p dz_{l+1}[p] accumulated in
// fp32; dW and db are finally scaled by 1 / (n out) in fp32.
//
// Kernels.
//  - train_fwd_kernel: a group of consecutive layers whose A fragments fit in
//    LDS, per wave 32-point tiles, the same register layer hand-off as the
//    fused MLP (mlp_layout.h); the hidden outputs the backward pass reads are
//    also stored (fp16, tile-fragment layout, below); the group that ends the
//    chain computes g = 2 (y - t) and per-block partial sums of (y - t)^2.
//    train_fwd_pair_kernel is the same with compile-time shapes and two
//    staggered tiles per wave.
//  - train_pair_kernel: layers l and l - 1 in one pass (pairs from the head
//    down): recomputes h_l from the stored h_{l-1}, keeps g_{l-1} in LDS, and
//    accumulates dW of both layers; only g_{l-2} reaches HBM.  The forward
//    therefore stores every other activation.
//  - train_bwd_kernel: dW and db of layer 0 alone (when the chain has an odd
//    number of layers); a block of 4 waves stages 32-point tiles of dz_1 and
//    the chain input in two LDS buffers (the next tile's loads in flight while
//    the current one is computed), then wave w computes one 32-row tile of dW
//    (K = the tile's points, operands gathered from the LDS tile); dW stays in
//    registers across the block's whole point range and is written once as a
//    per-block partial.
//  - train_reduce1/2_kernel: sum the per-block partials in a fixed order.
#include <algorithm>
#include <mutex>
#include <string>

#include "mlp_core.h"

namespace rdv {

constexpr int kTrMT = 4;      // 32-row M tiles per layer (widths <= 128)
constexpr int kTrKC = 8;      // 16-wide K chunks per layer
constexpr int kTrWaves = 8;   // forward block
constexpr int kTrFwdThreads = 64 * kTrWaves;
constexpr int kTrBwdThreads = 256;

struct TrainFwdArgs {
  const uint8_t* packed;
  MlpLayout lay;
  int L, l0, l1;                        // layers [l0, l1) of an L-layer chain
  const half_t* in;                     // layer l0's input: the chain input [n, in_w[0]] fp16 (l0 == 0), else tile-fragment layout
  half_t* hout[RDV_MLP_MAX_LAYERS];     // hout[l]: output of layer l (l < L - 1), tile-fragment layout, or null (not kept)
  const float* target;                  // [n, out] fp32 (l1 == L)
  half_t* g;                            // 2 (y - t), tile-fragment layout of width out (l1 == L)
  float* loss_partial;                  // [gridDim.x] (l1 == L)
  int64_t n;
  int has_bias;
};

// Sum over a wave (every lane gets it): DPP row shifts + row broadcasts.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float tr_dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, true));
}
__device__ __forceinline__ float tr_wave_sum(float v) {
  v += tr_dpp<0x111, 0xF>(v);
  v += tr_dpp<0x112, 0xF>(v);
  v += tr_dpp<0x114, 0xF>(v);
  v += tr_dpp<0x118, 0xF>(v);
  v += tr_dpp<0x142, 0xA>(v);
  v += tr_dpp<0x143, 0xC>(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

typedef half_t half4v __attribute__((ext_vector_type(4)));

// Tile-fragment layout of the step's intermediate fp16 buffers (the kept hidden
// activations h_i, the head gradient g and the gradients g_i between backward
// launches), [rows][W] with rows a multiple of 64: 32-point tiles of
// Wp = 16 ceil(W / 16) features, tile k at k 32 Wp; within a tile, 16-byte chunk
// c = 64 s + 32 hh + col holds point col, features 16 s + 4 hh + 0..3 and then
// 16 s + 8 + 4 hh + 0..3 (tfl_feature).  That chunk is lane 32 hh + col's B
// fragment of K chunk s in the hidden (chunk_sigma) order, and equally the fp16
// of D registers 8 (s % 2) .. + 7 of 32-row block s / 2, so a wave writes or
// reads a whole 1 KiB slot s with one 16-byte access per lane.  Features past W
// are stored as zeros.
__device__ __forceinline__ int tfl_feature(int s, int hh, int j) { return 16 * s + 4 * hh + (j & 3) + ((j >> 2) << 3); }

__global__ __launch_bounds__(kTrFwdThreads, 1) void train_fwd_kernel(TrainFwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ float s_loss[kTrWaves];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h = lane >> 5, col = lane & 31;
  const MlpLayout& lay = a.lay;
  // stage the group's fragments and biases: [frag bytes of l0..l1-1][bias floats]
  const int64_t fbase = lay.frag_off[a.l0];
  const int64_t fend = lay.frag_off[a.l1 - 1] + int64_t(lay.mt[a.l1 - 1]) * lay.kc[a.l1 - 1] * 1024;
  const int64_t bbase = lay.bias_off[a.l0];
  const int64_t bend = lay.bias_off[a.l1 - 1] + int64_t(lay.mt[a.l1 - 1]) * 128;
  {
    const uint4* src = reinterpret_cast<const uint4*>(a.packed + fbase);
    uint4* dst = reinterpret_cast<uint4*>(smem);
    for (int64_t i = threadIdx.x; i < (fend - fbase) / 16; i += blockDim.x) dst[i] = src[i];
    const uint4* bsrc = reinterpret_cast<const uint4*>(a.packed + bbase);
    uint4* bdst = reinterpret_cast<uint4*>(smem + (fend - fbase));
    for (int64_t i = threadIdx.x; i < (bend - bbase) / 16; i += blockDim.x) bdst[i] = bsrc[i];
  }
  __syncthreads();
  const half8* sw = reinterpret_cast<const half8*>(smem);
  const float* sb = reinterpret_cast<const float*>(smem + (fend - fbase));

  const int64_t ntiles = (a.n + 31) / 32;
  const int64_t per_block = (ntiles + gridDim.x - 1) / gridDim.x;
  const int64_t t_begin = int64_t(blockIdx.x) * per_block;
  const int64_t t_end = t_begin + per_block < ntiles ? t_begin + per_block : ntiles;
  const bool last_group = a.l1 == a.L;
  float loss = 0.0f;

  for (int64_t tile = t_begin + wave; tile < t_end; tile += kTrWaves) {
    const int64_t p = tile * 32 + col;            // this lane's point
    const bool pv = p < a.n;
    const int64_t pc = pv ? p : a.n - 1;          // clamped row for loads
    half8 b[kTrKC];
    {
      const int w0 = lay.in_w[a.l0];
      const int kc0 = lay.kc[a.l0];
      const half_t* row = a.in + pc * w0;
      const half8* slots = reinterpret_cast<const half8*>(a.in + tile * 32 * w0);
#pragma unroll
      for (int c = 0; c < kTrKC; ++c) {
        if (c < kc0) {
          // natural order (the chain input): features 16c + 8h + 0..7; a hidden
          // input: slot c of the tile-fragment layout
          b[c] = a.l0 == 0 ? *reinterpret_cast<const half8*>(row + 16 * c + 8 * h) : slots[c * 64 + lane];
        }
      }
    }
    for (int l = a.l0; l < a.l1; ++l) {
      const int mt = lay.mt[l], kc = lay.kc[l];
      const int frag = int((lay.frag_off[l] - fbase) / 16) / 64;  // first fragment of layer l in LDS
      const int boff = int((lay.bias_off[l] - bbase) / 4);        // first bias of layer l in LDS
      f32x16 acc[kTrMT];
#pragma unroll
      for (int t = 0; t < kTrMT; ++t) {
        if (t < mt) {
          if (a.has_bias) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f32x4 bv = *reinterpret_cast<const f32x4*>(sb + boff + 32 * t + 8 * q + 4 * h);
#pragma unroll
              for (int jj = 0; jj < 4; ++jj) acc[t][4 * q + jj] = bv[jj];
            }
          } else {
            acc[t] = f32x16{};
          }
        }
      }
#pragma unroll
      for (int c = 0; c < kTrKC; ++c) {
        if (c < kc) {
#pragma unroll
          for (int t = 0; t < kTrMT; ++t)
            if (t < mt)
              acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sw[(frag + t * kc + c) * 64 + lane], b[c], acc[t], 0, 0, 0);
        }
      }
      if (l == a.L - 1) {
        // head: y = D rows (32t + 8q + 4h + jj) < out; g = 2 (y - t), loss += (y - t)^2
        const int out = lay.out_w[l];
        const int wg = 16 * ((out + 15) / 16);
        half8* gs = reinterpret_cast<half8*>(a.g + tile * 32 * wg);
#pragma unroll
        for (int t = 0; t < kTrMT; ++t) {
          if (t < mt) {
#pragma unroll
            for (int qq = 0; qq < 2; ++qq) {
              if (32 * t + 16 * qq < out) {
                half8 gv;
#pragma unroll
                for (int hi = 0; hi < 2; ++hi) {
                  // registers 8qq + 4hi + jj: rows 32t + 16qq + 8hi + 4h + jj
                  const int r = 32 * t + 16 * qq + 8 * hi + 4 * h;
                  if (32 * t + 16 * qq + 8 * hi < out) {
                    const f32x4 tv = *reinterpret_cast<const f32x4*>(a.target + pc * out + r);
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                      const float d = acc[t][8 * qq + 4 * hi + jj] - tv[jj];
                      loss += pv ? d * d : 0.0f;
                      gv[4 * hi + jj] = half_t(d + d);
                    }
                  } else {
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) gv[4 * hi + jj] = half_t(0.0f);
                  }
                }
                gs[(2 * t + qq) * 64 + lane] = gv;
              }
            }
          }
        }
      } else {
        // ReLU, fp16: store the hidden output (slot 2t + qq of the tile) and hand it to the next layer
        const int out = lay.out_w[l];
        half8* dst = a.hout[l] == nullptr ? nullptr : reinterpret_cast<half8*>(a.hout[l] + tile * 32 * out);
#pragma unroll
        for (int t = 0; t < kTrMT; ++t) {
          if (t < mt) {
#pragma unroll
            for (int qq = 0; qq < 2; ++qq) {
              half8 v;
#pragma unroll
              for (int j = 0; j < 8; ++j) v[j] = half_t(acc[t][8 * qq + j]);
              v = __builtin_elementwise_max(v, half8{0, 0, 0, 0, 0, 0, 0, 0});
              b[2 * t + qq] = v;
              if (dst != nullptr) dst[(2 * t + qq) * 64 + lane] = v;
            }
          }
        }
      }
    }
  }
  if (last_group) {
    loss = tr_wave_sum(loss);
    if (lane == 0) s_loss[wave] = loss;
    __syncthreads();
    if (threadIdx.x == 0) {
      float s = 0.0f;
      for (int w = 0; w < kTrWaves; ++w) s += s_loss[w];
      a.loss_partial[blockIdx.x] = s;
    }
  }
}

// ------------------------------------------------- forward, tile pairs
// train_fwd_pair_kernel: the same group evaluation with a compile-time chain
// shape N (Net<RDV_ENC_NONE, in width, 0, out width, kc of the group's first
// layer, mt of each layer>).  Each wave evaluates 64 points at a time as two
// 32-point tiles A and B staggered by half a layer (stage_pair, mlp_core.h):
// one tile's fp32 -> fp16 hand-off runs between the other tile's MFMAs.  A
// kept activation is stored from the hand-off registers, one 1 KiB slot per
// store (tile-fragment layout).
//   KEEP: bit l set when the output of the group's layer l is stored
//         (a.hout[a.l0 + l]); NAT0: the group input is the chain input (natural
//         K order), else a stored hidden activation (chunk_sigma K order);
//   HEAD: the group ends the chain (g = 2 (y - t) and the loss partials).
// Buffers hold whole pair tiles (rows rounded up to 64), so every store is
// unconditional; rows >= n hold values never read as data.
template <class N, int l>
__device__ __forceinline__ void tf_store(const half8 (&b)[N::kMaxKC], half_t* tile_base, int lane) {
  half8* d = reinterpret_cast<half8*>(tile_base);
#pragma unroll
  for (int s = 0; s < 2 * N::mt(l); ++s) d[s * 64 + lane] = b[s];
}

// tA, tB: the two tiles' indices.
template <class N, int l, int KEEP, bool HEAD>
__device__ __forceinline__ void tf_layers(const LdsWeights& ws, const float* sb, int h, half8 (&bA)[N::kMaxKC],
                                          half8 (&bB)[N::kMaxKC], f32x16 (&accA)[N::kMaxMT],
                                          f32x16 (&accB)[N::kMaxMT], const TrainFwdArgs& a, int64_t tA, int64_t tB) {
  constexpr int L = N::kL;
  constexpr int W = 32 * N::mt(l);  // output width of a hidden layer
  const int lane = ws.lane;
  // stage boundaries are scheduling barriers: a stage holds the accumulators
  // of two tiles, never three
  __builtin_amdgcn_sched_barrier(0);
  load_bias<N, l>(accA, sb, h);
  if constexpr (l == 0) {
    stage_pair<N, 0, -1, true, true>(ws, bA, accA, accB, bB);
  } else {
    constexpr int Wp = 32 * N::mt(l - 1);
    stage_pair<N, l, l - 1, true, true>(ws, bA, accA, accB, bB);
    if constexpr ((KEEP >> (l - 1)) & 1) tf_store<N, l - 1>(bB, a.hout[a.l0 + l - 1] + tB * 32 * Wp, lane);
  }
  __builtin_amdgcn_sched_barrier(0);
  load_bias<N, l>(accB, sb, h);
  constexpr bool handA = l + 1 < L || !HEAD;
  stage_pair<N, l, handA ? l : -1, true, true>(ws, bB, accB, accA, bA);
  if constexpr (handA && ((KEEP >> l) & 1)) tf_store<N, l>(bA, a.hout[a.l0 + l] + tA * 32 * W, lane);
  if constexpr (l + 1 < L) {
    tf_layers<N, l + 1, KEEP, HEAD>(ws, sb, h, bA, bB, accA, accB, a, tA, tB);
  } else if constexpr (!HEAD) {
#pragma unroll
    for (int s = 0; s < 2 * N::mt(l); ++s) handoff_slot<N, l, true>(s, accB, bB);
    if constexpr ((KEEP >> l) & 1) tf_store<N, l>(bB, a.hout[a.l0 + l] + tB * 32 * W, lane);
  }
}

constexpr int kTfWaves = 8;  // two per SIMD
constexpr int kTfThreads = 64 * kTfWaves;

template <class N, int KEEP, bool HEAD, bool NAT0>
__global__ __launch_bounds__(kTfThreads, 1) void train_fwd_pair_kernel(TrainFwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ float s_loss[kTfWaves];
  constexpr int L = N::kL;
  constexpr int IN0 = N::kIn;
  constexpr int KC0 = N::kc(0);
  constexpr int OUT = N::kOut;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int h = lane >> 5, col = lane & 31;
  half8* sw = reinterpret_cast<half8*>(smem);
  float* sb = reinterpret_cast<float*>(smem + N::kFrags * 1024);

  const int64_t n = a.n;
  const int64_t npairs = (n + 63) / 64;
  const int64_t per_block = (npairs + gridDim.x - 1) / gridDim.x;
  const int64_t p_begin = int64_t(blockIdx.x) * per_block;
  const int64_t p_end = p_begin + per_block < npairs ? p_begin + per_block : npairs;

  // this lane's input fragments of tile `tile`: the chain input by rows (clamped;
  // rows >= n compute values that are never used), a hidden input by slots
  auto load_in = [&](int64_t tile, half8 (&b)[N::kMaxKC]) {
    int64_t row = tile * 32 + col;
    row = row < n - 1 ? row : n - 1;
    const half_t* src = a.in + row * IN0;
    const half8* slots = reinterpret_cast<const half8*>(a.in + tile * 32 * IN0);
#pragma unroll
    for (int c = 0; c < KC0; ++c) {
      if constexpr (NAT0) b[c] = *reinterpret_cast<const half8*>(src + 16 * c + 8 * h);
      else b[c] = slots[c * 64 + lane];
    }
  };
  half8 bA[N::kMaxKC], bB[N::kMaxKC];
  int64_t pt = p_begin + wave;
  if (pt < p_end) {
    load_in(2 * pt, bA);
    load_in(2 * pt + 1, bB);
  }
  // stage the group's fragments and biases (biases compacted to Net's bias_base),
  // eight 16-byte loads per thread in flight at a time
  stage_net_weights<N, kTfThreads, 8>(a.packed, a.lay, sb, sw, a.l0);
  __syncthreads();

  // narrow inputs (KC0 <= 4) are loaded a whole iteration ahead into spare
  // registers; wider ones at the end of the previous iteration, into bA / bB
  constexpr bool kEarly = KC0 <= 4;
  half8 nA[kEarly ? KC0 : 1], nB[kEarly ? KC0 : 1];
  float loss = 0.0f;
  for (; pt < p_end; pt += kTfWaves) {
    const int64_t pA = pt * 64 + col, pB = pA + 32;
    const int64_t nxt = pt + kTfWaves;
    if constexpr (kEarly) {
      if (nxt < p_end) {
        half8 fA[N::kMaxKC], fB[N::kMaxKC];
        load_in(2 * nxt, fA);
        load_in(2 * nxt + 1, fB);
#pragma unroll
        for (int c = 0; c < KC0; ++c) {
          nA[c] = fA[c];
          nB[c] = fB[c];
        }
      }
    }
    f32x16 accA[N::kMaxMT], accB[N::kMaxMT];
    const LdsWeights ws{sw + opaque_zero(), lane};
    tf_layers<N, 0, KEEP, HEAD>(ws, sb + opaque_zero(), h, bA, bB, accA, accB, a, 2 * pt, 2 * pt + 1);
    if constexpr (HEAD) {
      // y = D rows 32t + 16qq + 8hi + 4h + jj (registers 8qq + 4hi + jj) < OUT;
      // g = 2 (y - t) as slot 2t + qq of the tile, zero past OUT; loss over rows < n
      constexpr int WG = 16 * ((OUT + 15) / 16);
      const int64_t cA = pA < n ? pA : n - 1, cB = pB < n ? pB : n - 1;
      half8* gA = reinterpret_cast<half8*>(a.g + 2 * pt * 32 * WG);
      half8* gB = reinterpret_cast<half8*>(a.g + (2 * pt + 1) * 32 * WG);
#pragma unroll
      for (int t = 0; t < N::mt(L - 1); ++t) {
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          if (32 * t + 16 * qq < OUT) {
            half8 vA, vB;
#pragma unroll
            for (int hi = 0; hi < 2; ++hi) {
              const int r = 32 * t + 16 * qq + 8 * hi + 4 * h;
              if (32 * t + 16 * qq + 8 * hi < OUT) {
                const f32x4 tA = *reinterpret_cast<const f32x4*>(a.target + cA * OUT + r);
                const f32x4 tB = *reinterpret_cast<const f32x4*>(a.target + cB * OUT + r);
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                  const float dA = accA[t][8 * qq + 4 * hi + jj] - tA[jj];
                  const float dB = accB[t][8 * qq + 4 * hi + jj] - tB[jj];
                  loss += (pA < n ? dA * dA : 0.0f) + (pB < n ? dB * dB : 0.0f);
                  vA[4 * hi + jj] = half_t(dA + dA);
                  vB[4 * hi + jj] = half_t(dB + dB);
                }
              } else {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                  vA[4 * hi + jj] = half_t(0.0f);
                  vB[4 * hi + jj] = half_t(0.0f);
                }
              }
            }
            gA[(2 * t + qq) * 64 + lane] = vA;
            gB[(2 * t + qq) * 64 + lane] = vB;
          }
        }
      }
    }
    if constexpr (kEarly) {
#pragma unroll
      for (int c = 0; c < KC0; ++c) {
        bA[c] = nA[c];
        bB[c] = nB[c];
      }
    } else if (nxt < p_end) {
      load_in(2 * nxt, bA);
      load_in(2 * nxt + 1, bB);
    }
  }
  if constexpr (HEAD) {
    loss = tr_wave_sum(loss);
    if (lane == 0) s_loss[wave] = loss;
    __syncthreads();
    if (threadIdx.x == 0) {
      float s = 0.0f;
      for (int w = 0; w < kTfWaves; ++w) s += s_loss[w];
      a.loss_partial[blockIdx.x] = s;
    }
  }
}

// LDS bytes of train_fwd_pair_kernel<N, ...>.
template <class N>
constexpr int64_t tf_lds() {
  return int64_t(N::kFrags) * 1024 + int64_t(N::kBias) * 4;
}

// Specialisations: the two forward groups of the benchmark chain
// 32 -> 128 x 8 -> 16 (layers 0-4 and 5-8 under the 150 KiB LDS cap).
using TfNetC5a = Net<RDV_ENC_NONE, 32, 0, 128, 2, 4, 4, 4, 4, 4>;  // 32 -> 128 x 5, keeps h1, h3, h5
using TfNetC5b = Net<RDV_ENC_NONE, 128, 0, 16, 8, 4, 4, 4, 1>;     // 128 -> 128 x 3 -> 16, keeps h7

struct TfEntry {
  int in0, nat0, head, keep, L, out, kc0;
  int mt[RDV_MLP_MAX_LAYERS];
  const void* fn;
  int64_t lds;
};

template <class N, int KEEP, bool HEAD, bool NAT0>
TfEntry tf_entry() {
  TfEntry e{};
  e.in0 = N::kIn;
  e.nat0 = NAT0;
  e.head = HEAD;
  e.keep = KEEP;
  e.L = N::kL;
  e.out = N::kOut;
  e.kc0 = N::kc(0);
  for (int i = 0; i < N::kL; ++i) e.mt[i] = N::mt(i);
  e.fn = reinterpret_cast<const void*>(&train_fwd_pair_kernel<N, KEEP, HEAD, NAT0>);
  e.lds = tf_lds<N>();
  return e;
}

static const TfEntry* tf_table(int* count) {
  static const TfEntry table[] = {
      tf_entry<TfNetC5a, 0x15, false, true>(),
      tf_entry<TfNetC5b, 0x2, true, false>(),
  };
  *count = int(sizeof(table) / sizeof(table[0]));
  return table;
}

// --------------------------------------------------------------- backward
struct TrainBwdArgs {
  const half_t* dz;   // gradient of layer 0's output (pre-activation), tile-fragment layout of width out
  const half_t* hin;  // [n, in] the chain input
  float* dw_part;     // [gridDim.x][out][in]
  float* db_part;     // [gridDim.x][out]
  int in, out;
  int64_t n;
};

constexpr int kTrPad = 8;  // LDS row padding (halves): rows 8 points apart fall in different banks
constexpr int kTrLoads = 4;  // 16-byte loads per thread per tile: 32 x (128 + 128) halves / 256 threads

__global__ __launch_bounds__(kTrBwdThreads, 2) void train_bwd_kernel(TrainBwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h = lane >> 5, col = lane & 31;
  const int mto = (a.out + 31) / 32;       // dW row tiles (o)
  const int mti = (a.in + 31) / 32;        // dW column tiles (i)
  const int kco = (a.out + 15) / 16;       // 16-feature slots of dz
  const int OP = 32 * mto + kTrPad;        // LDS dz row stride (halves), columns >= out stay 0
  const int IP = 32 * mti + kTrPad;        // LDS h row stride (halves), columns >= in stay 0
  half_t* sdz = reinterpret_cast<half_t*>(smem);
  // zero both tile buffers (their padding columns stay zero)
  for (int i = threadIdx.x; i < 2 * 32 * (OP + IP); i += blockDim.x) sdz[i] = half_t(0.0f);
  __syncthreads();

  const int64_t ntiles = (a.n + 31) / 32;
  const int64_t per_block = (ntiles + gridDim.x - 1) / gridDim.x;
  const int64_t t_begin = int64_t(blockIdx.x) * per_block;
  const int64_t t_end = t_begin + per_block < ntiles ? t_begin + per_block : ntiles;

  const int to = __builtin_amdgcn_readfirstlane(wave);  // this wave's dW row tile (if < mto)
  __builtin_assume(to >= 0 && to < kTrBwdThreads / 64);
  f32x16 accw[kTrMT];
#pragma unroll
  for (int t = 0; t < kTrMT; ++t) accw[t] = f32x16{};
  float dbs = 0.0f;               // db of row 32 to + col, this lane's half of the points

  const int dz_chunks = 64 * kco;         // 16-byte chunks per tile
  const int h_chunks = 32 * a.in / 8;
  const int tile_halves = 32 * (OP + IP);
  // this thread's share of a tile's chunks (at most kTrLoads: widths <= 128);
  // dz chunk i is the tile's i-th 16 bytes (point i % 32, features
  // tfl_feature(i / 64, (i / 32) % 2, 0..7))
  auto load_tile = [&](int64_t tile, half8 (&r)[kTrLoads]) {
#pragma unroll
    for (int k = 0; k < kTrLoads; ++k) {
      const int i = k * kTrBwdThreads + int(threadIdx.x);
      half8 v = {};
      if (i < dz_chunks) {
        const int64_t p = tile * 32 + (i & 31);
        if (p < a.n) v = *reinterpret_cast<const half8*>(a.dz + tile * 32 * (16 * kco) + 8 * i);
      } else if (i < dz_chunks + h_chunks) {
        const int kk = i - dz_chunks;
        const int rr = kk / (a.in / 8), c8 = kk % (a.in / 8);
        const int64_t p = tile * 32 + rr;
        if (p < a.n) v = *reinterpret_cast<const half8*>(a.hin + p * a.in + 8 * c8);
      }
      r[k] = v;
    }
  };
  auto park_tile = [&](half_t* buf, const half8 (&r)[kTrLoads]) {
#pragma unroll
    for (int k = 0; k < kTrLoads; ++k) {
      const int i = k * kTrBwdThreads + int(threadIdx.x);
      if (i < dz_chunks) {
        const int f0 = tfl_feature(i >> 6, (i >> 5) & 1, 0);
        half_t* row = buf + (i & 31) * OP + f0;
        *reinterpret_cast<half4v*>(row) = half4v{r[k][0], r[k][1], r[k][2], r[k][3]};
        *reinterpret_cast<half4v*>(row + 8) = half4v{r[k][4], r[k][5], r[k][6], r[k][7]};
      } else if (i < dz_chunks + h_chunks) {
        const int kk = i - dz_chunks;
        const int rr = kk / (a.in / 8), c8 = kk % (a.in / 8);
        *reinterpret_cast<half8*>(buf + 32 * OP + rr * IP + 8 * c8) = r[k];
      }
    }
  };
  if (t_begin < t_end) {
    half8 r[kTrLoads];
    load_tile(t_begin, r);
    park_tile(sdz, r);
  }
  __syncthreads();
  for (int64_t tile = t_begin; tile < t_end; ++tile) {
    const int cur = int((tile - t_begin) & 1);
    const half_t* tdz = sdz + cur * tile_halves;
    const half_t* th = tdz + 32 * OP;
    // the next tile's loads are in flight while this tile is computed
    half8 r[kTrLoads];
    const bool more = tile + 1 < t_end;
    if (more) load_tile(tile + 1, r);

    // ---- dW rows tile to += dz^T[32 to .. +31][tile points] . h[tile points][:]
    if (to < mto) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        half8 af;
#pragma unroll
        for (int j = 0; j < 8; ++j) af[j] = tdz[(16 * ks + 8 * h + j) * OP + 32 * to + col];
#pragma unroll
        for (int j = 0; j < 8; ++j) dbs += float(af[j]);
#pragma unroll
        for (int t = 0; t < kTrMT; ++t) {
          if (t < mti) {
            half8 bf;
#pragma unroll
            for (int j = 0; j < 8; ++j) bf[j] = th[(16 * ks + 8 * h + j) * IP + 32 * t + col];
            accw[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, accw[t], 0, 0, 0);
          }
        }
      }
    }
    if (more) park_tile(sdz + (cur ^ 1) * tile_halves, r);  // the other buffer: last read a tile ago
    __syncthreads();
  }

  // ---- per-block partials: dW rows 32 to + 8q + 4h + jj, column 32 t + col
  if (to < mto) {
    float* dst = a.dw_part + int64_t(blockIdx.x) * a.out * a.in;
#pragma unroll
    for (int t = 0; t < kTrMT; ++t) {
      if (t < mti) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int o = 32 * to + 8 * q + 4 * h + jj;
            if (o < a.out && 32 * t + col < a.in) dst[int64_t(o) * a.in + 32 * t + col] = accw[t][4 * q + jj];
          }
      }
    }
    const float other = __shfl_xor(dbs, 32, 64);
    const int o = 32 * to + col;
    if (h == 0 && o < a.out) a.db_part[int64_t(blockIdx.x) * a.out + o] = dbs + other;
  }
}

// ------------------------------------------------------- backward, layer pairs
// Layers l and l - 1 in one pass over the points, so that neither the hidden
// activation h_l between them nor the gradient g_{l-1} ever reaches HBM:
//   h_l      = relu(fp16(W_{l-1} h_{l-1} + b_{l-1}))   recomputed, bit-identical to the forward
//   g_{l-1}  = fp16((g_l W_l) * [h_l > 0])              kept in LDS
//   dW_l    += g_l^T h_l,          db_l     += sum g_l
//   dW_{l-1}+= g_{l-1}^T h_{l-1},  db_{l-1} += sum g_{l-1}
//   g_{l-2}  = fp16((g_{l-1} W_{l-1}) * [h_{l-1} > 0])  written, unless l - 1 is the first layer
// Per 32-point tile the block stages g_l and h_{l-1} into LDS (the next tile's
// global loads in flight during the current one), and wave w computes the
// 32-row block w of every 128-wide product: the recompute (forward A fragments
// of layer l - 1, the same MFMA sequence as the forward), g_{l-1} (W_l^T
// fragments, masked with its own recomputed rows), the dW row blocks (K = the
// tile's points) and g_{l-2}.  dW of both layers stays in registers over the
// block's point range and is written once as a partial.
//
// LDS holds every tile twice: row-major [point][feature] (the operands whose K
// is a feature: 16-byte reads of 8 consecutive features of one point) and
// feature-major [feature][point] (the dW operands, whose K is the point: 8-byte
// reads of consecutive points of one feature).  Feature-major copies are written
// with 2-byte stores as tiles are parked or produced; their 36-half rows make
// both the stores and the 8-byte reads bank-conflict free.
struct TrainPairArgs {
  const half_t* g;       // g_l, tile-fragment layout of width out
  const half_t* hin;     // h_{l-1}: the chain input [n, in0] when l - 1 == 0, else tile-fragment layout
  const half_t* wf;      // layer l-1 forward A fragments [mid / 32][kc0][64][8] (packed layout)
  const float* bias;     // layer l-1 padded bias [mid]
  const half_t* wtl;     // W_l^T fragments [mid / 32][ceil(out / 16)][64][8]
  const half_t* wtl1;    // W_{l-1}^T fragments [in0 / 32][mid / 16][64][8] (gout only)
  half_t* gout;          // g_{l-2}, tile-fragment layout of width in0, or null
  float* dw_l;           // [gridDim.x][out][mid]
  float* db_l;           // [gridDim.x][out]
  float* dw_l1;          // [gridDim.x][mid][in0]
  float* db_l1;          // [gridDim.x][mid]
  int in0, mid, out;
  int kc0;               // K chunks of layer l - 1's forward fragments
  int natural0;          // layer l - 1 is layer 0: its K slots are in natural order (else chunk_sigma)
  int64_t n;
};

constexpr int kTpThreads = 512;  // 8 waves: two roles of 4
constexpr int kTpT = 36;         // feature-major row stride (halves)

// 8 consecutive halves of a feature-major row (8-byte aligned) as one fragment.
__device__ __forceinline__ half8 tp_frag(const half_t* p) {
  const half4v lo = *reinterpret_cast<const half4v*>(p);
  const half4v hi = *reinterpret_cast<const half4v*>(p + 4);
  return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// LDS carve-up of train_pair_kernel (halves; after the fp32 bias), per tile
// parity b: the inputs of the tile (row-major g_l, h_{l-1}; feature-major g_l,
// h_{l-1}) and the products (row-major g_{l-1}; feature-major g_{l-1}, h_l).
struct PairLds {
  int OP, IP, MP, in_halves, pr_halves;
  __device__ __host__ PairLds(int in0, int mid, int out) {
    const int mto = (out + 31) / 32, mti = (in0 + 31) / 32;
    OP = 32 * mto + kTrPad;
    IP = 32 * mti + kTrPad;
    MP = mid + kTrPad;
    in_halves = 32 * OP + 32 * IP + kTpT * (32 * mto + 32 * mti);
    pr_halves = 32 * MP + kTpT * 2 * mid;
  }
  __device__ __host__ int total_halves() const { return 2 * (in_halves + pr_halves); }
};

// Two roles, software-pipelined over the block's tiles (tile parity selects the
// LDS buffers):
//   waves 0-3, tile i:    h_l rows 32w.. (recompute) and g_{l-1} rows 32w..
//   waves 4-7, tile i-1:  dW_l, dW_{l-1} row blocks w, db, and g_{l-2} rows 32w..
// so each SIMD runs one wave of each, and the dW accumulators live only in the
// second role.  The weight fragments each wave needs (its 32-row blocks) sit in
// its registers.  Every iteration ends with two barriers around the parking of
// tile i+1 into the buffers tile i-1 used.
//
// IN0 / MID / OUT: the widths as compile-time constants (fully unrolled K loops),
// or 0 for the generic kernel that reads them from the arguments.  NAT0: the K
// order of layer l - 1's forward fragments (natural for layer 0, chunk_sigma
// after).  GOUT: 1 when g_{l-2} is written, 0 when not, -1 to read a.gout.
template <int IN0, int MID, int OUT, bool NAT0, int GOUT>
__global__ __launch_bounds__(kTpThreads, 1) void train_pair_kernel(TrainPairArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;
  const int in0 = IN0 ? IN0 : a.in0;
  const int mid = MID ? MID : a.mid;
  const int out = OUT ? OUT : a.out;
  const int mtm = mid / 32;              // row blocks of h_l and g_{l-1}
  const int mto = (out + 31) / 32;       // row blocks of dW_l
  const int mti = (in0 + 31) / 32;       // column blocks of dW_{l-1}
  const bool gout = GOUT < 0 ? a.gout != nullptr : GOUT != 0;
  const int mtg = gout ? in0 / 32 : 0;   // row blocks of g_{l-2}
  const int kco = (out + 15) / 16;
  const int kcm = mid / 16;
  const int kc0 = IN0 ? (NAT0 ? (IN0 + 15) / 16 : IN0 / 16) : a.kc0;
  constexpr int T = kTpT;
  const PairLds L(in0, mid, out);
  const int OP = L.OP, IP = L.IP, MP = L.MP;
  float* sbias = reinterpret_cast<float*>(smem);
  half_t* base = reinterpret_cast<half_t*>(sbias + mid);
  auto rg = [&](int b) { return base + b * (L.in_halves + L.pr_halves); };  // g_l [32][OP]
  auto rh = [&](int b) { return rg(b) + 32 * OP; };                         // h_{l-1} [32][IP]
  auto tg = [&](int b) { return rh(b) + 32 * IP; };                         // g_l^T [32 mto][T]
  auto th = [&](int b) { return tg(b) + T * 32 * mto; };                    // h_{l-1}^T [32 mti][T]
  auto rg1 = [&](int b) { return th(b) + T * 32 * mti; };                   // g_{l-1} [32][MP]
  auto tg1 = [&](int b) { return rg1(b) + 32 * MP; };                       // g_{l-1}^T [mid][T]
  auto thl = [&](int b) { return tg1(b) + T * mid; };                       // h_l^T [mid][T]
  for (int i = threadIdx.x; i < mid; i += blockDim.x) sbias[i] = a.bias[i];
  for (int i = threadIdx.x; i < L.total_halves(); i += blockDim.x) base[i] = half_t(0.0f);  // padding stays zero

  const int64_t ntiles = (a.n + 31) / 32;
  const int64_t per_block = (ntiles + gridDim.x - 1) / gridDim.x;
  const int64_t t_begin = int64_t(blockIdx.x) * per_block;
  const int64_t t_end = t_begin + per_block < ntiles ? t_begin + per_block : ntiles;
  const int count = int(t_end > t_begin ? t_end - t_begin : 0);
  // wave-uniform in scalar registers: role tests are scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  __builtin_assume(wave >= 0 && wave < kTpThreads / 64);
  const int role = wave >> 2, w = wave & 3;

  // Tile chunks (16 bytes of one point): chunk kk covers point kk % 32.  g_l and
  // a hidden h_{l-1} come in the tile-fragment layout (chunk kk is the tile's
  // kk-th 16 bytes: features tfl_feature(kk / 64, (kk / 32) % 2, 0..7)); the
  // chain input by rows (features 8 (kk / 32) + 0..7).  g_l's chunks first,
  // then h_{l-1}'s.  Consecutive lanes take consecutive points, so the
  // feature-major stores of a chunk fill consecutive halves of a row.
  constexpr int kLoads = 2;  // 16-byte chunks per thread: 32 x (128 + 128) halves / 512 threads
  const int g_chunks = 64 * kco;
  const int h_chunks = 32 * (in0 / 8);
  // Loads are unconditional (in-range rows or slots; unused slots re-read a valid
  // chunk) so that the compiler can count the wave's outstanding memory ops
  // exactly: a wait for these loads then never waits for the g_{l-2} stores
  // issued after them.  Points past n are zeroed when parked.
  __builtin_assume(threadIdx.x < kTpThreads);
  auto load_tile = [&](int64_t tile, half8 (&r)[kLoads]) {
#pragma unroll
    for (int k = 0; k < kLoads; ++k) {
      const int i = k * kTpThreads + int(threadIdx.x);
      const bool isg = i < g_chunks;
      const int kk = isg ? i : (i < g_chunks + h_chunks ? i - g_chunks : 0);
      const half_t* src;
      if (isg) {
        src = a.g + tile * 32 * (16 * kco) + 8 * kk;
      } else if (NAT0) {
        int64_t p = tile * 32 + (kk & 31);
        p = p < a.n ? p : a.n - 1;
        src = a.hin + p * in0 + 8 * (kk >> 5);
      } else {
        src = a.hin + tile * 32 * in0 + 8 * kk;
      }
      r[k] = *reinterpret_cast<const half8*>(src);
    }
  };
  auto park_tile = [&](int b, int64_t tile, const half8 (&r)[kLoads]) {
#pragma unroll
    for (int k = 0; k < kLoads; ++k) {
      const int i = k * kTpThreads + int(threadIdx.x);
      if (i < g_chunks + h_chunks) {
        const bool isg = i < g_chunks;
        const int kk = isg ? i : i - g_chunks;
        const int pp = kk & 31;
        const half8 v = tile * 32 + pp < a.n ? r[k] : half8{};
        half_t* rowp = isg ? rg(b) + pp * OP : rh(b) + pp * IP;
        half_t* t = (isg ? tg(b) : th(b)) + pp;
        if (isg || !NAT0) {
          // tile-fragment chunk: features f0 + 0..3 and f0 + 8 + 0..3
          const int f0 = tfl_feature(kk >> 6, (kk >> 5) & 1, 0);
          *reinterpret_cast<half4v*>(rowp + f0) = half4v{v[0], v[1], v[2], v[3]};
          *reinterpret_cast<half4v*>(rowp + f0 + 8) = half4v{v[4], v[5], v[6], v[7]};
#pragma unroll
          for (int j = 0; j < 8; ++j) t[(f0 + (j & 3) + ((j >> 2) << 3)) * T] = v[j];
        } else {
          const int f0 = 8 * (kk >> 5);
          *reinterpret_cast<half8*>(rowp + f0) = v;
#pragma unroll
          for (int j = 0; j < 8; ++j) t[(f0 + j) * T] = v[j];
        }
      }
    }
  };
  __syncthreads();  // zeroed buffers before the first park
  if (count > 0) {
    half8 r[kLoads];
    load_tile(t_begin, r);
    park_tile(0, t_begin, r);
  }
  __syncthreads();

  if (role == 0) {
    // ================= role 0: h_l and g_{l-1} of tile it (rows 32w..)
    half8 wf[kTrKC], wl[kTrKC];
#pragma unroll
    for (int c = 0; c < kTrKC; ++c) {
      wf[c] = (w < mtm && c < kc0) ? reinterpret_cast<const half8*>(a.wf)[(w * kc0 + c) * 64 + lane] : half8{};
      wl[c] = (w < mtm && c < kco) ? reinterpret_cast<const half8*>(a.wtl)[(w * kco + c) * 64 + lane] : half8{};
    }
    // all of them in registers before the loop, so that no wait inside it has
    // to cover these loads
    __builtin_amdgcn_s_waitcnt(0);
    for (int it = 0; it <= count; ++it) {
      half8 r[kLoads];
      const bool more = it + 1 < count;
      if (more) load_tile(t_begin + it + 1, r);
      if (it < count && w < mtm) {
        const int b = it & 1;
        const half_t* xh = rh(b);
        const half_t* xg = rg(b);
        f32x16 acc;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 bv = *reinterpret_cast<const f32x4*>(sbias + 32 * w + 8 * q + 4 * h);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) acc[4 * q + jj] = bv[jj];
        }
        // the forward's MFMA sequence for layer l - 1: h_l bit-identical
#pragma unroll
        for (int c = 0; c < kTrKC; ++c) {
          if (c < kc0) {
            half8 bf;
            if constexpr (NAT0) {
              bf = *reinterpret_cast<const half8*>(xh + col * IP + 16 * c + 8 * h);
            } else {
              const half4v lo = *reinterpret_cast<const half4v*>(xh + col * IP + 16 * c + 4 * h);
              const half4v hi = *reinterpret_cast<const half4v*>(xh + col * IP + 16 * c + 8 + 4 * h);
              bf = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[c], bf, acc, 0, 0, 0);
          }
        }
        f32x16 accg = {};
#pragma unroll
        for (int c = 0; c < kTrKC; ++c) {
          if (c < kco) {
            const half8 bf = *reinterpret_cast<const half8*>(xg + col * OP + 16 * c + 8 * h);
            accg = __builtin_amdgcn_mfma_f32_32x32x16_f16(wl[c], bf, accg, 0, 0, 0);
          }
        }
        // D register 4q + jj is feature 32w + 8q + 4h + jj of point col
        half_t* ohl = thl(b);
        half_t* og1 = rg1(b);
        half_t* ot1 = tg1(b);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          half4v hv, o;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) hv[jj] = half_t(acc[4 * q + jj]);
          hv = __builtin_elementwise_max(hv, half4v{0, 0, 0, 0});
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) o[jj] = float(hv[jj]) > 0.0f ? half_t(accg[4 * q + jj]) : half_t(0.0f);
          const int f = 32 * w + 8 * q + 4 * h;
          *reinterpret_cast<half4v*>(og1 + col * MP + f) = o;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            ohl[(f + jj) * T + col] = hv[jj];
            ot1[(f + jj) * T + col] = o[jj];
          }
        }
      }
      __syncthreads();  // tile it's products and tile it-1's reads complete
      if (more) park_tile((it + 1) & 1, t_begin + it + 1, r);
      __syncthreads();
    }
    return;
  }

  // ================= role 1: dW and g_{l-2} of tile it - 1 (row blocks w)
  half8 wl1[kTrKC];
#pragma unroll
  for (int c = 0; c < kTrKC; ++c)
    wl1[c] = (w < mtg && c < kcm) ? reinterpret_cast<const half8*>(a.wtl1)[(w * kcm + c) * 64 + lane] : half8{};
  __builtin_amdgcn_s_waitcnt(0);
  f32x16 accl[kTrMT], accl1[kTrMT];
#pragma unroll
  for (int t = 0; t < kTrMT; ++t) {
    accl[t] = f32x16{};
    accl1[t] = f32x16{};
  }
  float dbl = 0.0f, dbl1 = 0.0f;
  for (int it = 0; it <= count; ++it) {
    half8 r[kLoads];
    const bool more = it + 1 < count;
    if (more) load_tile(t_begin + it + 1, r);
    if (it >= 1) {
      const int b = (it - 1) & 1;
      const int64_t tile = t_begin + it - 1;
      // ---- dW_l rows 32w.. += g_l^T[32w.., points] h_l[points, :]
      if (w < mto) {
        const half_t* xtg = tg(b);
        const half_t* xhl = thl(b);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const half8 af = tp_frag(xtg + (32 * w + col) * T + 16 * ks + 8 * h);
#pragma unroll
          for (int j = 0; j < 8; ++j) dbl += float(af[j]);
#pragma unroll
          for (int t = 0; t < kTrMT; ++t) {
            if (t < mtm) {
              const half8 bf = tp_frag(xhl + (32 * t + col) * T + 16 * ks + 8 * h);
              accl[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, accl[t], 0, 0, 0);
            }
          }
        }
      }
      // ---- dW_{l-1} rows 32w.. += g_{l-1}^T[32w.., points] h_{l-1}[points, :]
      if (w < mtm) {
        const half_t* xt1 = tg1(b);
        const half_t* xth = th(b);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const half8 af = tp_frag(xt1 + (32 * w + col) * T + 16 * ks + 8 * h);
#pragma unroll
          for (int j = 0; j < 8; ++j) dbl1 += float(af[j]);
#pragma unroll
          for (int t = 0; t < kTrMT; ++t) {
            if (t < mti) {
              const half8 bf = tp_frag(xth + (32 * t + col) * T + 16 * ks + 8 * h);
              accl1[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, accl1[t], 0, 0, 0);
            }
          }
        }
      }
      // ---- g_{l-2} rows 32w.. = W_{l-1}^T[32w.., :] g_{l-1}^T, masked by h_{l-1} > 0
      if (w < mtg) {
        const half_t* xg1 = rg1(b);
        const half_t* xh = rh(b);
        f32x16 acc = {};
#pragma unroll
        for (int c = 0; c < kTrKC; ++c) {
          if (c < kcm) {
            const half8 bf = *reinterpret_cast<const half8*>(xg1 + col * MP + 16 * c + 8 * h);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(wl1[c], bf, acc, 0, 0, 0);
          }
        }
        // slots 2w + qq of the tile (registers 8qq + 0..7: features
        // tfl_feature(2w + qq, h, 0..7)); unconditional stores (exact wait counts)
        half8* dst = reinterpret_cast<half8*>(a.gout + tile * 32 * in0);
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          const int f0 = tfl_feature(2 * w + qq, h, 0);
          const half4v lo = *reinterpret_cast<const half4v*>(xh + col * IP + f0);
          const half4v hi = *reinterpret_cast<const half4v*>(xh + col * IP + f0 + 8);
          half8 o;
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            o[jj] = float(lo[jj]) > 0.0f ? half_t(acc[8 * qq + jj]) : half_t(0.0f);
            o[4 + jj] = float(hi[jj]) > 0.0f ? half_t(acc[8 * qq + 4 + jj]) : half_t(0.0f);
          }
          dst[(2 * w + qq) * 64 + lane] = o;
        }
      }
    }
    __syncthreads();  // tile it's products and tile it-1's reads complete
    if (more) park_tile((it + 1) & 1, t_begin + it + 1, r);
    __syncthreads();
  }

  // ---- per-block partials (rows 32w + 8q + 4h + jj, column 32t + col)
  if (w < mto) {
    float* dst = a.dw_l + int64_t(blockIdx.x) * out * mid;
#pragma unroll
    for (int t = 0; t < kTrMT; ++t)
      if (t < mtm)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int o = 32 * w + 8 * q + 4 * h + jj;
            if (o < out) dst[int64_t(o) * mid + 32 * t + col] = accl[t][4 * q + jj];
          }
    const float other = __shfl_xor(dbl, 32, 64);
    const int o = 32 * w + col;
    if (h == 0 && o < out) a.db_l[int64_t(blockIdx.x) * out + o] = dbl + other;
  }
  if (w < mtm) {
    float* dst = a.dw_l1 + int64_t(blockIdx.x) * mid * in0;
#pragma unroll
    for (int t = 0; t < kTrMT; ++t)
      if (t < mti)
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int o = 32 * w + 8 * q + 4 * h + jj;
            if (32 * t + col < in0) dst[int64_t(o) * in0 + 32 * t + col] = accl1[t][4 * q + jj];
          }
    const float other = __shfl_xor(dbl1, 32, 64);
    if (h == 0) a.db_l1[int64_t(blockIdx.x) * mid + 32 * w + col] = dbl1 + other;
  }
}

// All of a step's reductions in two launches, in a fixed order (so dW is the
// same run to run).  Job j sums its partials part_j[b][i] over b < nb_j into
// out_j[i] = scale * sum, i < count_j; the jobs' elements are concatenated
// (job j at start[j]) and so are their blocks (job j's first block bstart[j],
// 256 elements per block), so a block's job is wave-uniform.
//  stage 1: mid[s][e] = sum of part[b][i] for b = s, s + S, s + 2S, ... (in order)
//  stage 2: out[i] = scale * sum over s < S of mid[s][e] (in order)
constexpr int kTrSplit = 32;
constexpr int kTrMaxJobs = 2 * RDV_MLP_MAX_LAYERS + 1;
struct ReduceJobs {
  int n;
  const float* part[kTrMaxJobs];
  float* out[kTrMaxJobs];
  int nb[kTrMaxJobs];
  int64_t start[kTrMaxJobs + 1];
  int bstart[kTrMaxJobs + 1];
};

__device__ __forceinline__ int reduce_job(const ReduceJobs& J) {
  int j = 0;
  while (j + 1 < J.n && int(blockIdx.x) >= J.bstart[j + 1]) ++j;
  return j;
}

__global__ void train_reduce1_kernel(ReduceJobs J, float* __restrict__ mid) {
  const int j = reduce_job(J);
  const int64_t count = J.start[j + 1] - J.start[j];
  const int64_t i = int64_t(int(blockIdx.x) - J.bstart[j]) * 256 + threadIdx.x;
  if (i >= count) return;
  const int s = blockIdx.y;
  const float* part = J.part[j];
  float acc = 0.0f;
  for (int b = s; b < J.nb[j]; b += kTrSplit) acc += part[int64_t(b) * count + i];
  mid[int64_t(s) * J.start[J.n] + J.start[j] + i] = acc;
}

__global__ void train_reduce2_kernel(ReduceJobs J, const float* __restrict__ mid, float scale) {
  const int j = reduce_job(J);
  const int64_t count = J.start[j + 1] - J.start[j];
  const int64_t i = int64_t(int(blockIdx.x) - J.bstart[j]) * 256 + threadIdx.x;
  if (i >= count) return;
  const int64_t total = J.start[J.n];
  float acc = 0.0f;
#pragma unroll 8
  for (int s = 0; s < kTrSplit; ++s) acc += mid[int64_t(s) * total + J.start[j] + i];
  J.out[j][i] = acc * scale;
}

// Every transposed-weight pack of a step in one launch.  Job k writes the
// W^T fragments of one layer from its fp32 copy, element
// ((ti * kc + c) * 64 + lane) * 8 + j = W[o][32 ti + lane % 32] (zero past
// `out`), kc = ceil(out / 16), with o in the order of the kernel that reads it:
//   kTrPackWt  (train_pair_kernel):  o = 16 c + 8 (lane / 32) + j;
//   kTrPackWts (train_pair2_kernel): o = tfl_feature(c, lane / 32, j), the
//     tile-fragment K order; as an MFMA operand: rows (A) or columns (B)
//     32 ti .. of W^T, K = W's output features, chunk c.
enum { kTrPackWt = 0, kTrPackWts = 1 };
struct TrainPackJobs {
  const float* w32[RDV_MLP_MAX_LAYERS];
  half_t* wt[RDV_MLP_MAX_LAYERS];
  int in[RDV_MLP_MAX_LAYERS], out[RDV_MLP_MAX_LAYERS], kind[RDV_MLP_MAX_LAYERS];
  int64_t start[RDV_MLP_MAX_LAYERS + 1];  // first element of job k (start[n] = all elements)
  int n;
};

__global__ void train_pack_batch_kernel(TrainPackJobs J) {
  const int64_t g = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= J.start[J.n]) return;
  int k = 0;
  while (g >= J.start[k + 1]) ++k;
  const int64_t e = g - J.start[k];
  const int in = J.in[k], out = J.out[k];
  const int kc = (out + 15) / 16;
  const int j = int(e & 7);
  const int lane = int((e >> 3) & 63);
  const int64_t r = e >> 9;
  const int c = int(r % kc), ti = int(r / kc);
  const int o = J.kind[k] == kTrPackWts ? tfl_feature(c, lane >> 5, j) : 16 * c + 8 * (lane >> 5) + j;
  const int i = 32 * ti + (lane & 31);
  J.wt[k][e] = half_t(o < out ? J.w32[k][int64_t(o) * in + i] : 0.0f);
}

// ------------------------------------------ backward, layer pairs, point-major
// train_pair2_kernel: the layer pair of train_pair_kernel for 128-wide hidden
// layers l and l - 1 >= 1 (OUT = the width of g_l), with no operand gathered
// element by element.  The two products that read the tile put the points on
// the MFMA's M side, so their D registers hold, per lane, one feature over 16
// points: the layout of a K = points operand.
//   h_l     [points x m] = h_{l-1} W_{l-1}^T + b  (A: h_{l-1} slots, B: the forward's fragments)
//   g_{l-1} [points x m] = (g_l W_l) * [h_l > 0]   (A: g_l slots,     B: W_l^T, kTrPackWts order)
//   dW_l    [o x m]      += g_l^T h_l               (A: g_l^T,         B: h_l)
//   dW_{l-1}[m x i]      += g_{l-1}^T h_{l-1}       (A: g_{l-1},       B: h_{l-1}^T)
//   g_{l-2}^T [i x points] = W_{l-1}^T g_{l-1}^T, masked by h_{l-1} > 0, stored as slots
// Three operands change orientation: g_l and h_{l-1} (slots -> K = points) and
// g_{l-1} (K = points -> slots).  Each is an MFMA against a 0/1 selection
// fragment (tp2_select): every output is one fp16 value times 1 plus zeros,
// exact in fp32.  Wave w owns the 32-feature block w of every product and
// shares its block of the three through LDS as 1 KiB fragments.
//   Per tile: park (double-buffered slots of g_l, h_{l-1}), phase 1 (h_l, g_{l-1},
//   the three re-orientations, db), barrier, phase 2 (dW_l, dW_{l-1}, g_{l-2}),
//   the next tile's park, barrier.
// Points past n are parked as zeros: g_l = 0 there, so they add nothing.
struct TrainPair2Args {
  const half_t* g;     // g_l, tile-fragment layout of width OUT
  const half_t* hin;   // h_{l-1}, tile-fragment layout of width 128
  const half_t* wf;    // layer l-1 forward A fragments (packed layout)
  const float* bias;   // layer l-1 padded bias [128]
  const half_t* wls;   // W_l^T in the kTrPackWts order (in 128, out OUT)
  const half_t* wl1s;  // W_{l-1}^T in the kTrPackWts order (128 x 128)
  half_t* gout;        // g_{l-2}, tile-fragment layout of width 128
  float* dw_l;         // [gridDim.x][OUT][128]
  float* db_l;         // [gridDim.x][OUT]
  float* dw_l1;        // [gridDim.x][128][128]
  float* db_l1;        // [gridDim.x][128]
  int64_t n;
};

constexpr int kT2Threads = 512;  // 8 waves: two roles of 4

// 0/1 fragment par: lane (n = lane % 32, hh = lane / 32), element j is 1 where
// tfl_feature(par, hh, j) == n.  A x select(0) + A' x select(1) turns the K
// slots of two consecutive 16-feature chunks (or of the two 16-point halves of
// a K = points fragment pair) into the 32 columns of D.
__device__ __forceinline__ half8 tp2_select(int par, int lane) {
  half8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = tfl_feature(par, lane >> 5, j) == (lane & 31) ? half_t(1.0f) : half_t(0.0f);
  return v;
}

// D registers 8 ks .. 8 ks + 7 as fp16 (points tfl_feature(ks, h, 0..7) of a
// point-major product; features 32 block + tfl_feature(ks, h, 0..7) of a
// feature-major one).
__device__ __forceinline__ half8 tp2_half(const f32x16& d, int ks) {
  half8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = half_t(d[8 * ks + j]);
  return v;
}

// Sum of 8 fp16 values into an fp32 accumulator.
__device__ __forceinline__ float tp2_sum(const half8& v, float acc) {
#pragma unroll
  for (int j = 0; j < 8; j += 2) acc = __builtin_amdgcn_fdot2(half2v{v[j], v[j + 1]}, half2v{1, 1}, acc, false);
  return acc;
}

// LDS carve-up of train_pair2_kernel (half8 units): three input buffers
// (g_l slots, then h_{l-1} slots) and two exchange buffers (g_l and h_{l-1} as
// K = points fragments [block][ks][lane], g_{l-1} slots, h_l and g_{l-1} as
// K = points fragments).
template <int OUT>
struct Pair2Lds {
  static constexpr int KCO = (OUT + 15) / 16, MTO = (OUT + 31) / 32;
  static constexpr int kIn = 64 * (KCO + 8);
  static constexpr int kGT = 0, kHT = kGT + 2 * MTO * 64, kGP = kHT + 8 * 64, kHF = kGP + 8 * 64,
                       kGF = kHF + 8 * 64, kEx = kGF + 8 * 64;
  static constexpr int kBytes = (3 * kIn + 2 * kEx) * 16;
};

template <int OUT>
__global__ __launch_bounds__(kT2Threads, 1) void train_pair2_kernel(TrainPair2Args a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  using LD = Pair2Lds<OUT>;
  constexpr int KC = 8;                  // 16-feature chunks of a 128-wide layer
  constexpr int KCO = LD::KCO;           // chunks of g_l
  constexpr int MTO = LD::MTO;           // 32-row blocks of dW_l
  constexpr int kChunks = LD::kIn;       // 16-byte chunks per tile (g_l, then h_{l-1})
  constexpr int kLd = (kChunks + kT2Threads - 1) / kT2Threads;
  half8* const sIn = reinterpret_cast<half8*>(smem);
  half8* const sEx = sIn + 3 * LD::kIn;
  const int tid = int(threadIdx.x);
  const int lane = tid & 63;
  const int h = lane >> 5, col = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(wave >= 0 && wave < 8);
  __builtin_assume(tid < kT2Threads);
  const int role = wave >> 2, w = wave & 3;

  const int64_t ntiles = (a.n + 31) / 32;
  const int64_t per_block = (ntiles + gridDim.x - 1) / gridDim.x;
  const int64_t t_begin = int64_t(blockIdx.x) * per_block;
  const int64_t t_end = t_begin + per_block < ntiles ? t_begin + per_block : ntiles;
  const int count = int(t_end > t_begin ? t_end - t_begin : 0);

  // chunk i of a tile: g_l slot i / 64 (i < 64 KCO), else h_{l-1} slot (i - 64 KCO) / 64;
  // the chunk counts are multiples of 64, so a wave is all g_l or all h_{l-1}
  auto load = [&](int64_t tile, half8 (&r)[kLd]) {
#pragma unroll
    for (int k = 0; k < kLd; ++k) {
      const int i0 = k * kT2Threads + tid;
      const int i = i0 < kChunks ? i0 : 0;
      const half_t* src = i < 64 * KCO ? a.g + tile * 32 * (16 * KCO) + 8 * i
                                       : a.hin + tile * 32 * 128 + 8 * (i - 64 * KCO);
      r[k] = *reinterpret_cast<const half8*>(src);
    }
  };
  auto park = [&](int buf, int64_t tile, const half8 (&r)[kLd]) {
#pragma unroll
    for (int k = 0; k < kLd; ++k) {
      const int i = k * kT2Threads + tid;
      if (i < kChunks) sIn[buf * LD::kIn + i] = tile * 32 + (i & 31) < a.n ? r[k] : half8{};
    }
  };
  if (count > 0) {
    half8 r[kLd];
    load(t_begin, r);
    park(0, t_begin, r);
  }

  if (role == 0) {
    // ============ phase 1 of tile it: h_l, g_{l-1} of feature block w (point-major),
    // g_l and h_{l-1} block w to K = points fragments, g_{l-1} block w to slots
    half8 wf[KC], wl[KCO];
#pragma unroll
    for (int c = 0; c < KC; ++c) wf[c] = reinterpret_cast<const half8*>(a.wf)[(w * KC + c) * 64 + lane];
#pragma unroll
    for (int c = 0; c < KCO; ++c) wl[c] = reinterpret_cast<const half8*>(a.wls)[(w * KCO + c) * 64 + lane];
    f32x16 bias;  // D column 32w + col: the same bias in every register
    {
      const float bm = a.bias[32 * w + col];
#pragma unroll
      for (int q = 0; q < 16; ++q) bias[q] = bm;
    }
    const half8 sel0 = tp2_select(0, lane), sel1 = tp2_select(1, lane);
    float dbl = 0.0f, dbl1 = 0.0f;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (int it = 0; it <= count; ++it) {
      half8 r[kLd];
      const bool more = it + 1 < count;
      if (more) load(t_begin + it + 1, r);
      if (it < count) {
        const half8* G = sIn + (it % 3) * LD::kIn;
        const half8* H = G + 64 * KCO;
        half8* E = sEx + (it & 1) * LD::kEx;
        const half8 h0 = H[(2 * w) * 64 + lane], h1 = H[(2 * w + 1) * 64 + lane];
        f32x16 accR = __builtin_amdgcn_mfma_f32_32x32x16_f16(H[lane], wf[0], bias, 0, 0, 0);
#pragma unroll
        for (int c = 1; c < KC; ++c) accR = __builtin_amdgcn_mfma_f32_32x32x16_f16(H[c * 64 + lane], wf[c], accR, 0, 0, 0);
        f32x16 accG = {};
#pragma unroll
        for (int c = 0; c < KCO; ++c) accG = __builtin_amdgcn_mfma_f32_32x32x16_f16(G[c * 64 + lane], wl[c], accG, 0, 0, 0);
        f32x16 tH = {};
        tH = __builtin_amdgcn_mfma_f32_32x32x16_f16(h0, sel0, tH, 0, 0, 0);
        tH = __builtin_amdgcn_mfma_f32_32x32x16_f16(h1, sel1, tH, 0, 0, 0);
        E[LD::kHT + (2 * w) * 64 + lane] = tp2_half(tH, 0);
        E[LD::kHT + (2 * w + 1) * 64 + lane] = tp2_half(tH, 1);
        if (w < MTO) {
          f32x16 tG = {};
          tG = __builtin_amdgcn_mfma_f32_32x32x16_f16(G[(2 * w) * 64 + lane], sel0, tG, 0, 0, 0);
          if (2 * w + 1 < KCO)
            tG = __builtin_amdgcn_mfma_f32_32x32x16_f16(G[(2 * w + 1) * 64 + lane], sel1, tG, 0, 0, 0);
          const half8 g0 = tp2_half(tG, 0), g1 = tp2_half(tG, 1);
          E[LD::kGT + (2 * w) * 64 + lane] = g0;
          E[LD::kGT + (2 * w + 1) * 64 + lane] = g1;
          dbl = tp2_sum(g1, tp2_sum(g0, dbl));
        }
        // h_l = relu(fp16); g_{l-1} = fp16 where h_l > 0, i.e. where the
        // pre-activation exceeds 2^-25 (the largest value that rounds to 0)
        half8 gF[2];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          half8 hv = tp2_half(accR, ks);
          hv = __builtin_elementwise_max(hv, half8{0, 0, 0, 0, 0, 0, 0, 0});
          f32x16 gm;
#pragma unroll
          for (int j = 0; j < 8; ++j) gm[j] = accR[8 * ks + j] > 0x1p-25f ? accG[8 * ks + j] : 0.0f;
          half8 gv;
#pragma unroll
          for (int j = 0; j < 8; ++j) gv[j] = half_t(gm[j]);
          gF[ks] = gv;
          E[LD::kHF + (2 * w + ks) * 64 + lane] = hv;
          E[LD::kGF + (2 * w + ks) * 64 + lane] = gv;
          dbl1 = tp2_sum(gv, dbl1);
        }
        f32x16 tP = {};
        tP = __builtin_amdgcn_mfma_f32_32x32x16_f16(gF[0], sel0, tP, 0, 0, 0);
        tP = __builtin_amdgcn_mfma_f32_32x32x16_f16(gF[1], sel1, tP, 0, 0, 0);
        E[LD::kGP + (2 * w) * 64 + lane] = tp2_half(tP, 0);
        E[LD::kGP + (2 * w + 1) * 64 + lane] = tp2_half(tP, 1);
      }
      if (more) park((it + 1) % 3, t_begin + it + 1, r);
      __syncthreads();
    }
    // db partials: this lane's half of the points, feature 32w + col
    const float o0 = __shfl_xor(dbl, 32, 64);
    if (w < MTO && h == 0 && 32 * w + col < OUT) a.db_l[int64_t(blockIdx.x) * OUT + 32 * w + col] = dbl + o0;
    const float o1 = __shfl_xor(dbl1, 32, 64);
    if (h == 0) a.db_l1[int64_t(blockIdx.x) * 128 + 32 * w + col] = dbl1 + o1;
    return;
  }

  // ============ phase 2 of tile it - 1: dW_l[:, block w], dW_{l-1}[block w, :], g_{l-2} block w
  half8 wl1[KC];
#pragma unroll
  for (int c = 0; c < KC; ++c) wl1[c] = reinterpret_cast<const half8*>(a.wl1s)[(w * KC + c) * 64 + lane];
  f32x16 accL[MTO], accL1[4];
#pragma unroll
  for (int t = 0; t < MTO; ++t) accL[t] = f32x16{};
#pragma unroll
  for (int t = 0; t < 4; ++t) accL1[t] = f32x16{};
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int it = 0; it <= count; ++it) {
    half8 r[kLd];
    const bool more = it + 1 < count;
    if (more) load(t_begin + it + 1, r);
    if (it > 0) {
      const int64_t tile = t_begin + it - 1;
      const half8* H = sIn + ((it - 1) % 3) * LD::kIn + 64 * KCO;
      const half8* E = sEx + ((it - 1) & 1) * LD::kEx;
      const half8 hf0 = E[LD::kHF + (2 * w) * 64 + lane], hf1 = E[LD::kHF + (2 * w + 1) * 64 + lane];
      const half8 gf0 = E[LD::kGF + (2 * w) * 64 + lane], gf1 = E[LD::kGF + (2 * w + 1) * 64 + lane];
      f32x16 acc2 = {};
      if constexpr (MTO < 4) {
        // few dW_l products: each link of the g_{l-2} chain alternates with the
        // independent dW products (measured faster for the 16-wide head only)
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          acc2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(wl1[c], E[LD::kGP + c * 64 + lane], acc2, 0, 0, 0);
          const int ks = c & 1, blk = c >> 1;
          accL1[blk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ks ? gf1 : gf0, E[LD::kHT + c * 64 + lane], accL1[blk], 0, 0, 0);
          if (blk < MTO)
            accL[blk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(E[LD::kGT + c * 64 + lane], ks ? hf1 : hf0, accL[blk], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int ob = 0; ob < MTO; ++ob) {
          accL[ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(E[LD::kGT + (2 * ob) * 64 + lane], hf0, accL[ob], 0, 0, 0);
          accL[ob] = __builtin_amdgcn_mfma_f32_32x32x16_f16(E[LD::kGT + (2 * ob + 1) * 64 + lane], hf1, accL[ob], 0, 0, 0);
        }
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) {
          accL1[ib] = __builtin_amdgcn_mfma_f32_32x32x16_f16(gf0, E[LD::kHT + (2 * ib) * 64 + lane], accL1[ib], 0, 0, 0);
          accL1[ib] = __builtin_amdgcn_mfma_f32_32x32x16_f16(gf1, E[LD::kHT + (2 * ib + 1) * 64 + lane], accL1[ib], 0, 0, 0);
        }
#pragma unroll
        for (int c = 0; c < KC; ++c)
          acc2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(wl1[c], E[LD::kGP + c * 64 + lane], acc2, 0, 0, 0);
      }
      half8* dst = reinterpret_cast<half8*>(a.gout + tile * 32 * 128);
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
        const half8 hm = H[(2 * w + qq) * 64 + lane];  // h_{l-1}: the same features and point
        half8 o;
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = float(hm[j]) > 0.0f ? half_t(acc2[8 * qq + j]) : half_t(0.0f);
        dst[(2 * w + qq) * 64 + lane] = o;
      }
    }
    if (more) park((it + 1) % 3, t_begin + it + 1, r);
    __syncthreads();
  }
  {
    float* dst = a.dw_l + int64_t(blockIdx.x) * OUT * 128;
#pragma unroll
    for (int ob = 0; ob < MTO; ++ob)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int o = 32 * ob + 8 * (q >> 2) + 4 * h + (q & 3);  // D row of accL[ob]; column m = 32w + col
        if (o < OUT) dst[int64_t(o) * 128 + 32 * w + col] = accL[ob][q];
      }
  }
  {
    float* dst = a.dw_l1 + int64_t(blockIdx.x) * 128 * 128;
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
      for (int q = 0; q < 16; ++q) {
        const int m = 32 * w + 8 * (q >> 2) + 4 * h + (q & 3);  // D row of accL1[ib]; column i = 32ib + col
        dst[int64_t(m) * 128 + 32 * ib + col] = accL1[ib][q];
      }
  }
}

// ------------------------------------------------ backward, layer 0, point-major
// train_bwd0_kernel: dW_0 and db_0 for a 32-wide chain input and a 128-wide
// first layer.  dW_0[m][i] = sum_p g_0[p][m] x[p][i] with K = the points: wave
// w re-orients its 32-feature block of g_0 (slots 2w, 2w + 1) and the tile of
// x (two natural 16-feature chunks) with 0/1-fragment MFMAs, then accumulates
// its 32 x 32 block of dW_0.  No LDS: the four waves of a block walk the same
// tiles, each reading the tile's x (2 KiB) from L2.
constexpr int kB0Threads = 256;

// 0/1 fragment for the natural feature order of chunk par: lane (n, hh),
// element j is 1 where 16 par + 8 hh + j == n.
__device__ __forceinline__ half8 tp2_select_nat(int par, int lane) {
  half8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = 16 * par + 8 * (lane >> 5) + j == (lane & 31) ? half_t(1.0f) : half_t(0.0f);
  return v;
}

__global__ __launch_bounds__(kB0Threads, 2) void train_bwd0_kernel(TrainBwdArgs a) {
  const int tid = int(threadIdx.x);
  const int lane = tid & 63;
  const int h = lane >> 5, col = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(w >= 0 && w < 4);
  const int64_t ntiles = (a.n + 31) / 32;
  const int64_t per_block = (ntiles + gridDim.x - 1) / gridDim.x;
  const int64_t t_begin = int64_t(blockIdx.x) * per_block;
  const int64_t t_end = t_begin + per_block < ntiles ? t_begin + per_block : ntiles;
  const half8 sel0 = tp2_select(0, lane), sel1 = tp2_select(1, lane);
  const half8 nat0 = tp2_select_nat(0, lane), nat1 = tp2_select_nat(1, lane);
  // this lane's chunks of tile t: g_0 slots 2w, 2w + 1 and x row col, features 8h .. and 16 + 8h ..
  auto load = [&](int64_t t, half8 (&r)[4]) {
    const half8* gs = reinterpret_cast<const half8*>(a.dz + t * 32 * 128);
    r[0] = gs[(2 * w) * 64 + lane];
    r[1] = gs[(2 * w + 1) * 64 + lane];
    int64_t p = t * 32 + col;
    p = p < a.n ? p : a.n - 1;
    const half_t* xr = a.hin + p * 32;
    r[2] = *reinterpret_cast<const half8*>(xr + 8 * h);
    r[3] = *reinterpret_cast<const half8*>(xr + 16 + 8 * h);
  };
  f32x16 acc = {};
  float dbs = 0.0f;
  half8 cur[4];
  if (t_begin < t_end) load(t_begin, cur);
  for (int64_t t = t_begin; t < t_end; ++t) {
    half8 nxt[4];
    if (t + 1 < t_end) load(t + 1, nxt);
    // points past n: g_0 = 0 there (x is clamped, so finite)
    const bool valid = t * 32 + col < a.n;
    const half8 g0 = valid ? cur[0] : half8{}, g1 = valid ? cur[1] : half8{};
    f32x16 tg = {}, tx = {};
    tg = __builtin_amdgcn_mfma_f32_32x32x16_f16(g0, sel0, tg, 0, 0, 0);
    tg = __builtin_amdgcn_mfma_f32_32x32x16_f16(g1, sel1, tg, 0, 0, 0);
    tx = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[2], nat0, tx, 0, 0, 0);
    tx = __builtin_amdgcn_mfma_f32_32x32x16_f16(cur[3], nat1, tx, 0, 0, 0);
    // K = points fragments: lane = feature (m for g_0, i for x), registers = points
    const half8 ga = tp2_half(tg, 0), gb = tp2_half(tg, 1);
    const half8 xa = tp2_half(tx, 0), xb = tp2_half(tx, 1);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ga, xa, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(gb, xb, acc, 0, 0, 0);
    dbs = tp2_sum(gb, tp2_sum(ga, dbs));
#pragma unroll
    for (int k = 0; k < 4; ++k) cur[k] = nxt[k];
  }
  // partials: D row m = 32w + 8(q/4) + 4h + q%4, column i = col
  float* dst = a.dw_part + int64_t(blockIdx.x) * 128 * 32;
#pragma unroll
  for (int q = 0; q < 16; ++q) dst[int64_t(32 * w + 8 * (q >> 2) + 4 * h + (q & 3)) * 32 + col] = acc[q];
  const float other = __shfl_xor(dbs, 32, 64);
  if (h == 0) a.db_part[int64_t(blockIdx.x) * 128 + 32 * w + col] = dbs + other;
}

// ------------------------------------------------------------------- host
// Backward schedule: layer pairs (L-1, L-2), (L-3, L-4), ... through
// train_pair_kernel, then layer 0 alone (train_bwd_kernel, dW only) when L is
// odd.  The forward keeps h_i (the input of layer i) only where the backward
// or a later forward group reads it: i = L-2, L-4, ... >= 1, and the first
// layer of every forward group.
struct TrainPlan {
  int groups;
  int g0[RDV_MLP_MAX_LAYERS + 1];  // group k = layers [g0[k], g0[k + 1])
  int blocks_fwd, blocks_bwd, blocks_pair;
  bool keep[RDV_MLP_MAX_LAYERS];   // h_i stored by the forward
  int64_t wt_off[RDV_MLP_MAX_LAYERS], h_off[RDV_MLP_MAX_LAYERS], g_off, dz_off[2], dw_off[RDV_MLP_MAX_LAYERS],
      db_off[RDV_MLP_MAX_LAYERS], loss_off, mid_off;
  int64_t total;
};

static constexpr int64_t kTrFwdLdsCap = 150 * 1024;
static constexpr int64_t kTrPairLdsCap = 160 * 1024;

// Specialisations of train_pair_kernel: the layer pairs of the benchmark chain
// (128-wide hidden layers, a 16-wide head), then the generic kernel.
static const void* const kPairKernels[] = {
    reinterpret_cast<const void*>(&train_pair_kernel<128, 128, 128, false, 1>),
    reinterpret_cast<const void*>(&train_pair_kernel<128, 128, 16, false, 1>),
    reinterpret_cast<const void*>(&train_pair_kernel<0, 0, 0, false, -1>),
    reinterpret_cast<const void*>(&train_pair_kernel<0, 0, 0, true, -1>),
};

static const void* pair_kernel(const TrainPairArgs& pa) {
  const bool g = pa.gout != nullptr;
  if (g && !pa.natural0 && pa.in0 == 128 && pa.mid == 128 && pa.out == 128) return kPairKernels[0];
  if (g && !pa.natural0 && pa.in0 == 128 && pa.mid == 128 && pa.out == 16) return kPairKernels[1];
  return kPairKernels[pa.natural0 ? 3 : 2];
}

// LDS bytes of train_pair_kernel (same carve-up as the kernel).
static int64_t pair_lds(int in0, int mid, int out, int kc0, bool gout) {
  (void)kc0;
  (void)gout;
  const PairLds L(in0, mid, out);
  return int64_t(mid) * 4 + int64_t(L.total_halves()) * 2;
}

// train_fwd_pair_kernel instantiation for forward group [fa.l0, fa.l1), or nullptr.
static const TfEntry* find_tf(const rdv_mlp_desc& d, const MlpLayout& lay, const TrainFwdArgs& fa) {
  const int L = d.n_layers;
  int keep = 0;
  for (int i = fa.l0; i < fa.l1; ++i)
    if (fa.hout[i] != nullptr) keep |= 1 << (i - fa.l0);
  int nt = 0;
  const TfEntry* t = tf_table(&nt);
  for (int k = 0; k < nt; ++k) {
    const TfEntry& e = t[k];
    if (e.L != fa.l1 - fa.l0 || e.in0 != d.dims[fa.l0] || e.nat0 != (fa.l0 == 0) || e.head != (fa.l1 == L) ||
        e.keep != keep || e.out != d.dims[fa.l1])
      continue;
    bool ok = true;
    for (int i = 0; i < e.L && ok; ++i) ok = e.mt[i] == lay.mt[fa.l0 + i];
    if (e.kc0 != lay.kc[fa.l0]) ok = false;
    if (ok) return &e;
  }
  return nullptr;
}

static int64_t group_lds(const MlpLayout& lay, int l0, int l1) {
  int64_t f = 0, b = 0;
  for (int l = l0; l < l1; ++l) {
    f += int64_t(lay.mt[l]) * lay.kc[l] * 1024;
    b += int64_t(lay.mt[l]) * 128;
  }
  return f + b;
}

int train_check(const rdv_mlp_desc& d, const MlpLayout& lay) {
  const int L = d.n_layers;
  if (L < 2) return fail(RDV_ERR_UNSUPPORTED, "the training step needs at least two layers");
  if (d.encoding != RDV_ENC_NONE) return fail(RDV_ERR_UNSUPPORTED, "the training step takes raw (unencoded) inputs");
  for (int l = 0; l < L; ++l) {
    if (d.prec[l] != RDV_PREC_F16) return fail(RDV_ERR_UNSUPPORTED, "the training step runs LinearFast (fp16) layers");
    if (d.act[l] != (l + 1 < L ? RDV_ACT_RELU : RDV_ACT_NONE))
      return fail(RDV_ERR_UNSUPPORTED, "the training step needs ReLU hidden layers and a linear head");
  }
  if (d.dims[0] % 16 || d.dims[0] > 128) return fail(RDV_ERR_UNSUPPORTED, "input width must be a multiple of 16, <= 128");
  for (int l = 1; l < L; ++l)
    if (d.dims[l] % 32 || d.dims[l] > 128)
      return fail(RDV_ERR_UNSUPPORTED, "hidden widths must be multiples of 32, <= 128");
  if (d.dims[L] % 8 || d.dims[L] > 128) return fail(RDV_ERR_UNSUPPORTED, "output width must be a multiple of 8, <= 128");
  for (int l = 0; l < L; ++l)
    if (group_lds(lay, l, l + 1) > kTrFwdLdsCap) return fail(RDV_ERR_UNSUPPORTED, "layer too large for LDS");
  for (int l = L - 1; l >= 1; l -= 2)
    if (pair_lds(d.dims[l - 1], d.dims[l], d.dims[l + 1], lay.kc[l - 1], l - 1 > 0) > kTrPairLdsCap)
      return fail(RDV_ERR_UNSUPPORTED, "layer pair too large for LDS");
  return RDV_OK;
}

static void train_plan(const rdv_mlp_desc& d, const MlpLayout& lay, int64_t n, int cu, TrainPlan* p) {
  const int L = d.n_layers;
  p->groups = 0;
  int l = 0;
  while (l < L) {
    int e = l + 1;
    while (e < L && group_lds(lay, l, e + 1) <= kTrFwdLdsCap) ++e;
    p->g0[p->groups++] = l;
    l = e;
  }
  p->g0[p->groups] = L;
  const int64_t ntiles = (n + 31) / 32;
  p->blocks_fwd = int(std::min<int64_t>(cu, (ntiles + kTrWaves - 1) / kTrWaves));
  p->blocks_bwd = int(std::min<int64_t>(2 * int64_t(cu), ntiles));
  p->blocks_pair = int(std::max<int64_t>(1, std::min<int64_t>(cu, ntiles)));
  for (int i = 0; i < RDV_MLP_MAX_LAYERS; ++i) p->keep[i] = false;
  for (int i = L - 2; i >= 1; i -= 2) p->keep[i] = true;
  for (int k = 1; k < p->groups; ++k) p->keep[p->g0[k]] = true;
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t o = off;
    off = align256(off + bytes);
    return o;
  };
  int maxw = 0;
  for (int i = 0; i < L; ++i) {
    p->wt_off[i] = take(int64_t(d.dims[i] / 32 > 0 ? d.dims[i] / 32 : 1) * ((d.dims[i + 1] + 15) / 16) * 1024);
    maxw = std::max(maxw, d.dims[i]);
  }
  // tile-fragment buffers: whole pair tiles (rows rounded up to 64), widths padded to 16
  const int64_t rows = (n + 63) / 64 * 64;
  for (int i = 0; i < L; ++i) p->h_off[i] = (i >= 1 && p->keep[i]) ? take(rows * d.dims[i] * 2) : -1;
  p->g_off = take(rows * ((d.dims[L] + 15) / 16 * 16) * 2);
  p->dz_off[0] = take(rows * maxw * 2);
  p->dz_off[1] = take(rows * maxw * 2);
  // per-layer partials, all reduced together at the end of the step
  const int64_t parts = std::max(p->blocks_bwd, p->blocks_pair);
  int64_t all = 1;  // the loss
  for (int i = 0; i < L; ++i) {
    p->dw_off[i] = take(parts * d.dims[i + 1] * d.dims[i] * 4);
    p->db_off[i] = take(parts * d.dims[i + 1] * 4);
    all += int64_t(d.dims[i + 1]) * (d.dims[i] + 1);
  }
  p->loss_off = take(int64_t(p->blocks_fwd) * 4);
  p->mid_off = take(int64_t(kTrSplit) * all * 4);
  p->total = off;
}

int64_t train_workspace_bytes(const rdv_mlp_desc& d, const MlpLayout& lay, int64_t n, int cu) {
  TrainPlan p;
  train_plan(d, lay, n, cu, &p);
  return p.total;
}

int launch_train_step(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, const void* x,
                      const float* target, int64_t n, void* workspace, int64_t ws_bytes, float* loss,
                      float* const* dW, float* const* db, hipStream_t stream) {
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  TrainPlan p;
  train_plan(d, lay, n, di.cu_count, &p);
  if (ws_bytes < p.total) return fail(RDV_ERR_WORKSPACE, "training workspace too small");
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const int L = d.n_layers;
  const uint8_t* pk = static_cast<const uint8_t*>(packed);
  // forward groups
  static bool attr_set = false;
  if (!attr_set) {
    RDV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&train_fwd_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(kTrFwdLdsCap)));
    RDV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&train_bwd_kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 80 * 1024));
    for (const void* fn : kPairKernels)
      RDV_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(kTrPairLdsCap)));
    RDV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&train_pair2_kernel<128>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, Pair2Lds<128>::kBytes));
    RDV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&train_pair2_kernel<16>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, Pair2Lds<16>::kBytes));
    int nt = 0;
    const TfEntry* tt = tf_table(&nt);
    for (int k = 0; k < nt; ++k)
      RDV_HIP_TRY(hipFuncSetAttribute(tt[k].fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(tt[k].lds)));
    attr_set = true;
  }
  TrainFwdArgs fa;
  fa.packed = pk;
  fa.lay = lay;
  fa.L = L;
  fa.target = target;
  fa.g = reinterpret_cast<half_t*>(ws + p.g_off);
  fa.loss_partial = reinterpret_cast<float*>(ws + p.loss_off);
  fa.n = n;
  fa.has_bias = 1;  // the packed header's flag is on the device; biases are staged either way
  for (int i = 0; i < RDV_MLP_MAX_LAYERS; ++i) fa.hout[i] = nullptr;
  for (int i = 0; i + 1 < L; ++i)
    if (p.keep[i + 1]) fa.hout[i] = reinterpret_cast<half_t*>(ws + p.h_off[i + 1]);
  for (int k = 0; k < p.groups; ++k) {
    fa.l0 = p.g0[k];
    fa.l1 = p.g0[k + 1];
    fa.in = fa.l0 == 0 ? static_cast<const half_t*>(x) : reinterpret_cast<const half_t*>(ws + p.h_off[fa.l0]);
    const TfEntry* e = find_tf(d, lay, fa);
    if (e != nullptr) {
      void* args[] = {&fa};
      RDV_HIP_TRY(hipLaunchKernel(e->fn, dim3(unsigned(p.blocks_fwd)), dim3(kTfThreads), args, size_t(e->lds), stream));
    } else {
      const int64_t lds = group_lds(lay, fa.l0, fa.l1);
      train_fwd_kernel<<<dim3(unsigned(p.blocks_fwd)), dim3(kTrFwdThreads), size_t(lds), stream>>>(fa);
    }
    RDV_HIP_TRY(hipGetLastError());
  }
  const float scale = 1.0f / float(double(n) * d.dims[L]);
  ReduceJobs jobs;
  jobs.n = 0;
  jobs.start[0] = 0;
  jobs.bstart[0] = 0;
  // queues the reduction of part[nb][count] into out (run after the backward)
  auto reduce = [&](const float* part, int nb, int64_t count, float* out) -> int {
    const int j = jobs.n++;
    jobs.part[j] = part;
    jobs.out[j] = out;
    jobs.nb[j] = nb;
    jobs.start[j + 1] = jobs.start[j] + count;
    jobs.bstart[j + 1] = jobs.bstart[j] + int((count + 255) / 256);
    return RDV_OK;
  };
  rc = reduce(reinterpret_cast<float*>(ws + p.loss_off), p.blocks_fwd, 1, loss);
  if (rc != RDV_OK) return rc;
  // backward: layer pairs from the head down, then layer 0 alone if L is odd;
  // gradients ping-pong between dz_off[0] and dz_off[1]
  // The pair kernels' transposed weights, every layer >= 1 in the order its
  // pair kernel reads, packed in one launch before the first of them.
  auto use_pair2 = [&](int l) {
    return l - 1 >= 1 && d.dims[l - 1] == 128 && d.dims[l] == 128 && (d.dims[l + 1] == 128 || d.dims[l + 1] == 16);
  };
  auto wt_of = [&](int l) { return reinterpret_cast<half_t*>(ws + p.wt_off[l]); };
  {
    TrainPackJobs pj;
    pj.n = 0;
    pj.start[0] = 0;
    auto add = [&](int l, int kind) {
      const int k = pj.n++;
      pj.w32[k] = reinterpret_cast<const float*>(pk + lay.w32_off[l]);
      pj.wt[k] = wt_of(l);
      pj.in[k] = d.dims[l];
      pj.out[k] = d.dims[l + 1];
      pj.kind[k] = kind;
      pj.start[k + 1] = pj.start[k] + int64_t(d.dims[l] / 32) * ((d.dims[l + 1] + 15) / 16) * 64 * 8;
    };
    for (int l = L - 1; l >= 1; l -= 2) {
      const int kind = use_pair2(l) ? kTrPackWts : kTrPackWt;
      add(l, kind);
      if (l - 1 >= 1) add(l - 1, kind);
    }
    if (pj.n > 0 && pj.start[pj.n] > 0) {
      train_pack_batch_kernel<<<dim3(unsigned((pj.start[pj.n] + 255) / 256)), dim3(256), 0, stream>>>(pj);
      RDV_HIP_TRY(hipGetLastError());
    }
  }
  const half_t* gsrc = reinterpret_cast<const half_t*>(ws + p.g_off);
  int dst = 0;
  int l = L - 1;
  for (; l >= 1; l -= 2) {
    if (use_pair2(l)) {
      // point-major pair kernel
      TrainPair2Args pa;
      pa.g = gsrc;
      pa.hin = reinterpret_cast<const half_t*>(ws + p.h_off[l - 1]);
      pa.wf = reinterpret_cast<const half_t*>(pk + lay.frag_off[l - 1]);
      pa.bias = reinterpret_cast<const float*>(pk + lay.bias_off[l - 1]);
      pa.wls = wt_of(l);
      pa.wl1s = wt_of(l - 1);
      pa.gout = reinterpret_cast<half_t*>(ws + p.dz_off[dst]);
      pa.dw_l = reinterpret_cast<float*>(ws + p.dw_off[l]);
      pa.db_l = reinterpret_cast<float*>(ws + p.db_off[l]);
      pa.dw_l1 = reinterpret_cast<float*>(ws + p.dw_off[l - 1]);
      pa.db_l1 = reinterpret_cast<float*>(ws + p.db_off[l - 1]);
      pa.n = n;
      const dim3 grid(unsigned(p.blocks_pair)), block(kT2Threads);
      if (d.dims[l + 1] == 128)
        train_pair2_kernel<128><<<grid, block, size_t(Pair2Lds<128>::kBytes), stream>>>(pa);
      else
        train_pair2_kernel<16><<<grid, block, size_t(Pair2Lds<16>::kBytes), stream>>>(pa);
      RDV_HIP_TRY(hipGetLastError());
      const int out = d.dims[l + 1];
      rc = reduce(pa.dw_l, p.blocks_pair, int64_t(out) * 128, dW[l]);
      if (rc != RDV_OK) return rc;
      rc = reduce(pa.db_l, p.blocks_pair, out, db[l]);
      if (rc != RDV_OK) return rc;
      rc = reduce(pa.dw_l1, p.blocks_pair, int64_t(128) * 128, dW[l - 1]);
      if (rc != RDV_OK) return rc;
      rc = reduce(pa.db_l1, p.blocks_pair, 128, db[l - 1]);
      if (rc != RDV_OK) return rc;
      gsrc = pa.gout;
      dst ^= 1;
      continue;
    }
    TrainPairArgs pa;
    pa.in0 = d.dims[l - 1];
    pa.mid = d.dims[l];
    pa.out = d.dims[l + 1];
    pa.kc0 = lay.kc[l - 1];
    pa.natural0 = l - 1 == 0 ? 1 : 0;
    pa.n = n;
    pa.g = gsrc;
    pa.hin = l - 1 == 0 ? static_cast<const half_t*>(x) : reinterpret_cast<const half_t*>(ws + p.h_off[l - 1]);
    pa.wf = reinterpret_cast<const half_t*>(pk + lay.frag_off[l - 1]);
    pa.bias = reinterpret_cast<const float*>(pk + lay.bias_off[l - 1]);
    pa.wtl = wt_of(l);
    pa.wtl1 = l - 1 > 0 ? wt_of(l - 1) : nullptr;
    pa.gout = l - 1 > 0 ? reinterpret_cast<half_t*>(ws + p.dz_off[dst]) : nullptr;
    pa.dw_l = reinterpret_cast<float*>(ws + p.dw_off[l]);
    pa.db_l = reinterpret_cast<float*>(ws + p.db_off[l]);
    pa.dw_l1 = reinterpret_cast<float*>(ws + p.dw_off[l - 1]);
    pa.db_l1 = reinterpret_cast<float*>(ws + p.db_off[l - 1]);
    const size_t lds = size_t(pair_lds(pa.in0, pa.mid, pa.out, pa.kc0, pa.gout != nullptr));
    const void* fn = pair_kernel(pa);
    void* args[] = {&pa};
    RDV_HIP_TRY(hipLaunchKernel(fn, dim3(unsigned(p.blocks_pair)), dim3(kTpThreads), args, lds, stream));
    RDV_HIP_TRY(hipGetLastError());
    rc = reduce(pa.dw_l, p.blocks_pair, int64_t(pa.out) * pa.mid, dW[l]);
    if (rc != RDV_OK) return rc;
    rc = reduce(pa.db_l, p.blocks_pair, pa.out, db[l]);
    if (rc != RDV_OK) return rc;
    rc = reduce(pa.dw_l1, p.blocks_pair, int64_t(pa.mid) * pa.in0, dW[l - 1]);
    if (rc != RDV_OK) return rc;
    rc = reduce(pa.db_l1, p.blocks_pair, pa.mid, db[l - 1]);
    if (rc != RDV_OK) return rc;
    if (pa.gout != nullptr) {
      gsrc = pa.gout;
      dst ^= 1;
    }
  }
  if (l == 0) {
    // layer 0 alone: dW_0 = g_0^T x, no input gradient
    const int in = d.dims[0], out = d.dims[1];
    const int kco = (out + 15) / 16;
    const int mti = (in + 31) / 32, mto = (out + 31) / 32;
    TrainBwdArgs ba;
    ba.dz = gsrc;
    ba.hin = static_cast<const half_t*>(x);
    ba.dw_part = reinterpret_cast<float*>(ws + p.dw_off[0]);
    ba.db_part = reinterpret_cast<float*>(ws + p.db_off[0]);
    ba.in = in;
    ba.out = out;
    ba.n = n;
    if (in == 32 && out == 128) {
      train_bwd0_kernel<<<dim3(unsigned(p.blocks_bwd)), dim3(kB0Threads), 0, stream>>>(ba);
    } else {
      const size_t lds = 2 * (size_t(32) * (32 * mto + kTrPad) * 2 + size_t(32) * (32 * mti + kTrPad) * 2);
      train_bwd_kernel<<<dim3(unsigned(p.blocks_bwd)), dim3(kTrBwdThreads), lds, stream>>>(ba);
    }
    (void)kco;
    RDV_HIP_TRY(hipGetLastError());
    rc = reduce(ba.dw_part, p.blocks_bwd, int64_t(out) * in, dW[0]);
    if (rc != RDV_OK) return rc;
    rc = reduce(ba.db_part, p.blocks_bwd, out, db[0]);
    if (rc != RDV_OK) return rc;
  }
  float* mid = reinterpret_cast<float*>(ws + p.mid_off);
  const unsigned gx = unsigned(jobs.bstart[jobs.n]);
  train_reduce1_kernel<<<dim3(gx, kTrSplit), dim3(256), 0, stream>>>(jobs, mid);
  RDV_HIP_TRY(hipGetLastError());
  train_reduce2_kernel<<<dim3(gx), dim3(256), 0, stream>>>(jobs, mid, scale);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

}  // namespace rdv

// ------------------------------------------------ no-allocation variant
// rdv_mlp_train_step_static: the training step with its workspace in a
// file-scope device array instead of a caller buffer, for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops).  Each
// GPU the library runs on holds its own copy of the array until the process
// ends; every call on that GPU shares it, so calls that overlap on one GPU
// race.  Nothing in it has to start at zero: every launch of the step writes
// each partial it later reads (blocks without tiles write zero partials).
namespace rdv {

constexpr int64_t kTrainScratchBytes = RDV_TRAIN_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kTrainScratchBytes];

// Device address of this GPU's copy of `scratch`, resolved once per device with
// that device current.  The array's name is only a host-side stand-in: kernels
// get this address, never the name.
static int scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = 0;
  RDV_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(RDV_ERR_UNSUPPORTED, "device index out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(RDV_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    addr[dev] = p;
  }
  *out = addr[dev];
  return RDV_OK;
}

int launch_train_step_static(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, const void* x,
                             const float* target, int64_t n, float* loss, float* const* dW, float* const* db,
                             hipStream_t stream) {
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  TrainPlan p;
  train_plan(d, lay, n, di.cu_count, &p);
  if (p.total > kTrainScratchBytes)
    return fail(RDV_ERR_WORKSPACE, "rdv_mlp_train_step_static: this chain and n need " + std::to_string(p.total) +
                                       " bytes of workspace, more than the " + std::to_string(kTrainScratchBytes) +
                                       "-byte static scratch (use rdv_mlp_train_step with a caller workspace)");
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc != RDV_OK) return rc;
  return launch_train_step(d, lay, packed, x, target, n, ws, kTrainScratchBytes, loss, dW, db, stream);
}

}  // namespace rdv
