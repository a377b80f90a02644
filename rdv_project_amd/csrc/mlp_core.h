// Device-side core of the fused fp16 MLP: the compile-time network shape, the
// layer-0 input fragments (raw or frequency-encoded), the MFMA layer chain with
// the D -> B fragment hand-off, and the output heads.  Shared by the fused MLP
// kernel (mlp_fused.hip) and the MLP-in-the-loop renderer (render.hip).
//
// Fragment layout (mlp_layout.h): v_mfma_f32_32x32x16_f16 with the transposed
// formulation H^T = W X^T, 32 points per N block; lane l holds point l % 32 and
// feature half h = l / 32 of every K chunk.
#ifndef RDV_MLP_CORE_H
#define RDV_MLP_CORE_H

#include "mlp_layout.h"
#include "rdv_common.h"

namespace rdv {

template <int ENC, int IN, int OCT, int OUT, int KC0, int... MT>
struct Net {
  static constexpr int kEnc = ENC, kIn = IN, kOct = OCT, kOut = OUT;
  static constexpr int kL = sizeof...(MT);
  static constexpr int kMT[kL] = {MT...};
  static constexpr int mt(int l) { return kMT[l]; }
  static constexpr int kc(int l) { return l == 0 ? KC0 : 2 * kMT[l - 1]; }
  static constexpr int frag_base(int l) {
    int s = 0;
    for (int i = 0; i < l; ++i) s += kc(i) * mt(i);
    return s;
  }
  static constexpr int bias_base(int l) {
    int s = 0;
    for (int i = 0; i < l; ++i) s += 32 * mt(i);
    return s;
  }
  static constexpr int max_mt() {
    int m = 0;
    for (int i = 0; i < kL; ++i) m = mt(i) > m ? mt(i) : m;
    return m;
  }
  static constexpr int max_kc() {
    int m = 0;
    for (int i = 0; i < kL; ++i) m = kc(i) > m ? kc(i) : m;
    return m;
  }
  static constexpr int kFrags = frag_base(kL);
  static constexpr int kBias = bias_base(kL);
  static constexpr int kMaxMT = max_mt();
  static constexpr int kMaxKC = max_kc();
};

// ----------------------------------------------------------------- input
// Builds layer 0's B fragments for this lane's point from its raw input p.
template <class N>
__device__ __forceinline__ void build_input(const float (&p)[N::kIn], int h, half8 (&b)[N::kMaxKC]) {
  constexpr int D = N::kIn;
  if constexpr (N::kEnc == RDV_ENC_FREQ) {
    constexpr int L = N::kOct;
    constexpr int H0 = (L + 1) / 2;  // octaves of half 0 (freq_octaves_half0)
    constexpr int H1 = L - H0;
    // First octave of this lane half from the hardware sine/cosine, the rest by
    // the double-angle recurrence sin 2x = 2 sin x cos x, cos 2x = 1 - 2 sin^2 x
    // (3 VALU ops per octave instead of two quarter-rate transcendentals).
    // v_sin/v_cos take revolutions: sin(2^k pi p) = sin(2 pi * 2^(k-1) p), and
    // the power-of-two scale is exact.  Two doublings grow the ~1e-7 absolute
    // error of v_sin/v_cos to a few 1e-7, far below the fp16 rounding applied next.
    float sn[D][H0], cs[D][H0];
    const float scale = h ? __builtin_ldexpf(1.0f, H0 - 1) : 0.5f;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const float arg = scale * p[d];
      sn[d][0] = __builtin_amdgcn_sinf(arg);
      cs[d][0] = __builtin_amdgcn_cosf(arg);
#pragma unroll
      for (int i = 1; i < H0; ++i) {
        const float u = sn[d][i - 1] + sn[d][i - 1];
        sn[d][i] = u * cs[d][i - 1];
        cs[d][i] = __builtin_fmaf(-u, sn[d][i - 1], 1.0f);
      }
    }
#pragma unroll
    for (int c = 0; c < N::kc(0); ++c) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int s = 8 * c + j;
        float v = 0.0f;
        if (s < 2 * D * H0) {
          const int i = s / (2 * D), r = s % (2 * D);
          const bool is_cos = r >= D;
          const int d = is_cos ? r - D : r;
          v = is_cos ? cs[d][i] : sn[d][i];
          if (i >= H1) v = h ? 0.0f : v;
        } else if (s < 2 * D * H0 + D) {
          v = h ? 0.0f : p[s - 2 * D * H0];
        }
        b[c][j] = half_t(v);
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < N::kc(0); ++c) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int f0 = 16 * c + j, f1 = 16 * c + 8 + j;
        const float v0 = f0 < D ? p[f0 < D ? f0 : 0] : 0.0f;
        const float v1 = f1 < D ? p[f1 < D ? f1 : 0] : 0.0f;
        b[c][j] = half_t(h ? v1 : v0);
      }
    }
  }
}

// ----------------------------------------------------------------- layers
// Accumulators of layer l start at its bias: rows 32t + 8q + 4h + 0..3 of D are
// contiguous in the padded bias, one ds_read_b128 each.
template <class N, int l>
__device__ __forceinline__ void load_bias(f32x16 (&acc)[N::kMaxMT], const float* sb, int h) {
#pragma unroll
  for (int t = 0; t < N::mt(l); ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 bv = *reinterpret_cast<const f32x4*>(sb + N::bias_base(l) + 32 * t + 8 * q + 4 * h);
      acc[t][4 * q + 0] = bv[0];
      acc[t][4 * q + 1] = bv[1];
      acc[t][4 * q + 2] = bv[2];
      acc[t][4 * q + 3] = bv[3];
    }
  }
}

// Copies the A fragments and biases of layers l0 .. l0 + N::kL - 1 into LDS
// (fragment f at sw[64 f ..], bias b at sb[b], the compact order of
// Net::frag_base / bias_base).  The fragments are one contiguous region from
// frag_off[l0] (every layer's block is a multiple of 1 KiB, so the 256-byte
// alignment adds no gaps).  Global loads go out BATCH per thread before their
// LDS writes (all of them by default), so the copy costs a memory latency per
// batch rather than one per layer and array.
template <class N, int THREADS, int BATCH = (N::kFrags * 64 + THREADS - 1) / THREADS>
__device__ __forceinline__ void stage_net_weights(const uint8_t* packed, const MlpLayout& lay, float* sb, half8* sw,
                                                  int l0 = 0) {
  constexpr int kF = N::kFrags * 64;
  constexpr int kFPer = (kF + THREADS - 1) / THREADS;
  constexpr int kBPer = (N::kBias + THREADS - 1) / THREADS;
  const int tid = int(threadIdx.x);
  // biases: element i of layer q lives at bias_off[l0 + q] + 4 (i - bias_base(q))
  float b[kBPer];
#pragma unroll
  for (int k = 0; k < kBPer; ++k) {
    const int i0 = k * THREADS + tid;
    const int i = i0 < N::kBias ? i0 : N::kBias - 1;
    int64_t off = lay.bias_off[l0];
#pragma unroll
    for (int q = 1; q < N::kL; ++q)
      if (i >= N::bias_base(q)) off = lay.bias_off[l0 + q] - 4 * int64_t(N::bias_base(q));
    b[k] = *reinterpret_cast<const float*>(packed + off + 4 * int64_t(i));
  }
  const half8* fsrc = reinterpret_cast<const half8*>(packed + lay.frag_off[l0]);
#pragma unroll
  for (int k0 = 0; k0 < kFPer; k0 += BATCH) {
    half8 f[BATCH];
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const int i = (k0 + k) * THREADS + tid;
      if (k0 + k < kFPer) f[k] = fsrc[i < kF ? i : kF - 1];
    }
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const int i = (k0 + k) * THREADS + tid;
      if (k0 + k < kFPer && i < kF) sw[i] = f[k];
    }
  }
#pragma unroll
  for (int k = 0; k < kBPer; ++k) {
    const int i = k * THREADS + tid;
    if (i < N::kBias) sb[i] = b[k];
  }
}

// Shapes of stage_net_weights_direct for a compile-time network whose hidden
// widths are whole 32-row tiles (the host checks that: direct_fused_ok): layer
// q's weights are copied, fp32, into an LDS staging area with a row stride of
// pitch(q) floats -- the columns the layer reads plus padding that spreads a
// fragment read's 32 rows over the banks -- and the fragments are then built
// from there.
template <class N, int THREADS>
struct DirectStage {
  static constexpr int kCols0 = N::kEnc == RDV_ENC_FREQ ? N::kIn * (1 + 2 * N::kOct) : N::kIn;
  static constexpr int cols(int q) { return q == 0 ? kCols0 : 32 * N::mt(q - 1); }
  static constexpr int rows(int q) { return q == N::kL - 1 ? N::kOut : 32 * N::mt(q); }
  static constexpr int pitch(int q) { return q == 0 ? kCols0 + 1 : cols(q) + 4; }
  static constexpr int base(int q) {
    int s = 0;
    for (int i = 0; i < q; ++i) s += rows(i) * pitch(i);
    return s;
  }
  static constexpr int kFloats = base(N::kL);
  // loads: layer 0 one float per element, later layers one float4
  static constexpr int items(int q) { return q == 0 ? rows(0) * kCols0 : rows(q) * cols(q) / 4; }
  static constexpr int load_iters(int q) { return (items(q) + THREADS - 1) / THREADS; }
  static constexpr int units(int q) { return N::mt(q) * N::kc(q) * 64; }
  static constexpr int unit_iters(int q) { return (units(q) + THREADS - 1) / THREADS; }
};

// layer0_slot_feature for a compile-time network, by slot s = 8c + j of lane
// half hh: a FREQ half's trig slots hold, octave after octave, D sines then D
// cosines, which is the encoded feature order itself, so feature = D + 2D
// (first octave of the half) + s with no division; half 0 then holds p.
template <class N>
__device__ __forceinline__ int layer0_slot_feature_of(int s, int hh) {
  constexpr int D = N::kIn;
  if constexpr (N::kEnc != RDV_ENC_FREQ) {
    return 16 * (s >> 3) + 8 * hh + (s & 7);
  } else {
    constexpr int L = N::kOct, H0 = (L + 1) / 2;
    const int nh = hh ? L - H0 : H0, kbase = hh ? H0 : 0;
    if (s < 2 * D * nh) return D + 2 * D * kbase + s;
    return (hh == 0 && s < 2 * D * H0 + D) ? s - 2 * D * H0 : -1;
  }
}

// Copy of layer Q's weights into the staging area: coalesced global loads
// (consecutive threads, consecutive elements), all issued before the writes.
template <class N, int THREADS, int Q>
__device__ __forceinline__ void direct_copy_layer(const DirectWeights& dw, const MlpLayout& lay, float* st) {
  using S = DirectStage<N, THREADS>;
  constexpr int I = S::items(Q), K = S::load_iters(Q), C = S::cols(Q);
  const int tid = int(threadIdx.x);
  const float* W = dw.W[Q];
  if constexpr (Q == 0) {
    const int in_w = lay.in_w[0];
    float v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int e0 = k * THREADS + tid;
      const int e = e0 < I ? e0 : I - 1;
      const int m = e / C, col = e - m * C;
      v[k] = W[int64_t(m) * in_w + col];
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int e = k * THREADS + tid;
      if (e < I) {
        const int m = e / C, col = e - m * C;
        st[S::base(0) + m * S::pitch(0) + col] = v[k];
      }
    }
  } else {
    constexpr int C4 = C / 4;
    f32x4 v[K];
    if ((reinterpret_cast<uintptr_t>(W) & 15) == 0) {
      const f32x4* W4 = reinterpret_cast<const f32x4*>(W);
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int e0 = k * THREADS + tid;
        v[k] = W4[e0 < I ? e0 : I - 1];  // rows are exactly C floats: the flat float4 index
      }
    } else {  // a buffer off 16-byte alignment: the same elements, one float at a time
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const int e0 = k * THREADS + tid;
        const float* p = W + 4 * int64_t(e0 < I ? e0 : I - 1);
        v[k] = f32x4{p[0], p[1], p[2], p[3]};
      }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const int e = k * THREADS + tid;
      if (e < I) {
        const int m = e / C4, c4 = e - m * C4;
        *reinterpret_cast<f32x4*>(st + S::base(Q) + m * S::pitch(Q) + 4 * c4) = v[k];
      }
    }
  }
}

// Fragment units of layer Q from the staging area (the packer's slot mapping,
// mlp_pack.hip): a hidden layer's unit is two runs of four consecutive columns
// (the chunk_sigma quartets), two 16-byte reads; layer 0's follow its encoding.
template <class N, int THREADS, int Q>
__device__ __forceinline__ void direct_build_layer(const float* st, half8* sw) {
  using S = DirectStage<N, THREADS>;
  constexpr int U = S::units(Q), K = S::unit_iters(Q);
  const int tid = int(threadIdx.x);
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const int u = k * THREADS + tid;
    if (u < U) {
      const int f = u >> 6, lane = u & 63;
      const int t = f / N::kc(Q), c = f - t * N::kc(Q);
      const int m = 32 * t + (lane & 31), hh = lane >> 5;
      const bool row_ok = m < S::rows(Q);
      const float* r = st + S::base(Q) + (row_ok ? m : 0) * S::pitch(Q);
      half8 v;
      if constexpr (Q == 0) {
        // Slots past the row's kCols0 columns (a raw input narrower than its
        // 16-wide K chunk) are zero: the staging row holds only those columns
        // and its pitch padding is never written, so reading on would pick up
        // a neighbour row or whatever an earlier kernel left in the LDS (a
        // value beyond fp16 range turns 0 * Inf into NaN, which ReLU then
        // maps to 0 for every point).
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int ka = layer0_slot_feature_of<N>(8 * c + j, hh);
          const bool ok = row_ok && ka >= 0 && ka < S::kCols0;
          const float x = r[ok ? ka : 0];
          v[j] = half_t(ok ? x : 0.0f);
        }
      } else {
        const int col0 = 16 * c + 4 * hh;  // columns col0 .. +3 and col0 + 8 .. +11
        const f32x4 lo = *reinterpret_cast<const f32x4*>(r + col0);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(r + col0 + 8);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[j] = half_t(row_ok ? lo[j] : 0.0f);
          v[4 + j] = half_t(row_ok ? hi[j] : 0.0f);
        }
      }
      sw[N::frag_base(Q) * 64 + u] = v;
    }
  }
}

template <class N, int THREADS, int Q>
struct DirectLayers {
  __device__ __forceinline__ static void copy(const DirectWeights& dw, const MlpLayout& lay, float* st) {
    direct_copy_layer<N, THREADS, Q>(dw, lay, st);
    if constexpr (Q + 1 < N::kL) DirectLayers<N, THREADS, Q + 1>::copy(dw, lay, st);
  }
  __device__ __forceinline__ static void build(const float* st, half8* sw) {
    direct_build_layer<N, THREADS, Q>(st, sw);
    if constexpr (Q + 1 < N::kL) DirectLayers<N, THREADS, Q + 1>::build(st, sw);
  }
};

// stage_net_weights for parameters read straight from the layers' fp32 buffers
// (no packed block): the weights are copied into the staging area `st`
// (DirectStage::kFloats floats), then every fragment unit is built from there.
// Returns whether any of this thread's biases is non-zero (the block ORs them
// in place of the packer's header flags).  Contains a block barrier.
template <class N, int THREADS>
__device__ __forceinline__ bool stage_net_weights_direct(const DirectWeights& dw, const MlpLayout& lay, float* sb,
                                                         half8* sw, float* st) {
  constexpr int kBPer = (N::kBias + THREADS - 1) / THREADS;
  const int tid = int(threadIdx.x);
  float b[kBPer];
#pragma unroll
  for (int k = 0; k < kBPer; ++k) {
    const int i0 = k * THREADS + tid;
    const int i = i0 < N::kBias ? i0 : N::kBias - 1;
    int q = 0;
#pragma unroll
    for (int qq = 1; qq < N::kL; ++qq)
      if (i >= N::bias_base(qq)) q = qq;
    const float* Bq = dw.b[0];
    int bb = 0;
#pragma unroll
    for (int qq = 1; qq < N::kL; ++qq)
      if (q == qq) {
        Bq = dw.b[qq];
        bb = N::bias_base(qq);
      }
    const int o = i - bb;
    const bool ok = o < lay.out_w[q];
    b[k] = Bq[ok ? o : 0];
    b[k] = ok ? b[k] : 0.0f;
  }
  DirectLayers<N, THREADS, 0>::copy(dw, lay, st);
  __syncthreads();
  DirectLayers<N, THREADS, 0>::build(st, sw);
  bool nz = false;
#pragma unroll
  for (int k = 0; k < kBPer; ++k) {
    const int i = k * THREADS + tid;
    if (i < N::kBias) {
      sb[i] = b[k];
      nz = nz || b[k] != 0.0f;
    }
  }
  return nz;
}

// A wave's view of the block's LDS copy of the A fragments: fragment f is a
// conflict-free 1 KiB line, one ds_read_b128 per lane, read right before its MFMA.
struct LdsWeights {
  const half8* sw;  // fragment f at sw[f * 64 + lane]
  int lane;
  __device__ __forceinline__ half8 get(int f) const { return sw[f * 64 + lane]; }
};

// The same with fragments F0 .. F0 + NR - 1 held in registers for the life of
// the wave (read from LDS once): an MFMA whose A operand needs no LDS read
// leaves the LDS to the others (reads and MFMAs of a CU contend).  The index
// is a compile-time constant after unrolling, so the choice costs nothing.
template <int F0, int NR>
struct RegLdsWeights {
  const half8* sw;
  int lane;
  half8 r[NR > 0 ? NR : 1];
  __device__ __forceinline__ half8 get(int f) const { return (f >= F0 && f < F0 + NR) ? r[f - F0] : sw[f * 64 + lane]; }
};

// BIAS: the accumulators were seeded with the bias; otherwise the first K
// chunk starts from MFMA's zero C operand (all biases zero: nothing to load).
template <class N, int l, bool BIAS, class WS>
__device__ __forceinline__ void mfma_layer(const WS& ws, const half8 (&b)[N::kMaxKC], f32x16 (&acc)[N::kMaxMT]) {
  const f32x16 zero = {};
#pragma unroll
  for (int c = 0; c < N::kc(l); ++c) {
#pragma unroll
    for (int t = 0; t < N::mt(l); ++t) {
      const f32x16& cin = (BIAS || c > 0) ? acc[t] : zero;
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ws.get(N::frag_base(l) + t * N::kc(l) + c), b[c], cin, 0, 0, 0);
    }
  }
}

// D registers of layer l -> B fragments of layer l + 1 (hidden activations are
// all ReLU or all none on this path; the dispatcher routes anything else to the
// generic kernel).
template <class N, int l, bool RELU>
__device__ __forceinline__ void to_next(const f32x16 (&acc)[N::kMaxMT], half8 (&b)[N::kMaxKC]) {
  const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int t = 0; t < N::mt(l); ++t) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      half8 v;
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = half_t(acc[t][8 * q + j]);
      // max after the fp16 rounding equals rounding after max (rounding is monotone)
      if constexpr (RELU) v = __builtin_elementwise_max(v, zero);
      b[2 * t + q] = v;
    }
  }
}

// Layer l accumulates into `cur` (already holding its bias) while the next
// layer's bias is read into `nxt`; the two sets alternate down the chain, so
// every LDS read has a whole layer of matrix work to hide behind.  The last
// layer's result ends in acc set (kL - 1) % 2.
template <class N, int l, bool RELU, bool BIAS, class WS>
__device__ __forceinline__ void run_chain(const WS& ws, half8 (&b)[N::kMaxKC], f32x16 (&cur)[N::kMaxMT],
                                          f32x16 (&nxt)[N::kMaxMT], const float* sb, int h) {
  if constexpr (BIAS) {
    if constexpr (l + 1 < N::kL) load_bias<N, l + 1>(nxt, sb, h);
    // keep the machine scheduler from sinking those reads back to their use
    __builtin_amdgcn_sched_barrier(0);
  }
  mfma_layer<N, l, BIAS>(ws, b, cur);
  if constexpr (l + 1 < N::kL) {
    to_next<N, l, RELU>(cur, b);
    run_chain<N, l + 1, RELU, BIAS>(ws, b, nxt, cur, sb, h);
  }
}

// ------------------------------------------------------------ tile pairs
// Two 32-point tiles A and B per wave, staggered by half a layer: the MFMAs of
// one tile's layer l are interleaved, in program order, with the other tile's
// register hand-off (fp32 -> fp16 conversion and ReLU), which does not depend
// on them.  MFMA and VALU time on a SIMD overlap only when independent VALU
// work is ready while the matrix core is busy; this puts it right behind each
// MFMA of the wave itself.
//   stage l.a: layer l MFMAs of A  +  layer l-1 hand-off of B (B's input encoding at l = 0)
//   stage l.b: layer l MFMAs of B  +  layer l hand-off of A

// Hand-off slot s = 2t + q of layer lp: acc[t][8q .. 8q+7] -> b[s].
template <class N, int lp, bool RELU>
__device__ __forceinline__ void handoff_slot(int s, const f32x16 (&acc)[N::kMaxMT], half8 (&b)[N::kMaxKC]) {
  const int t = s >> 1, q = s & 1;
  half8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = half_t(acc[t][8 * q + j]);
  // max after the fp16 rounding equals rounding after max (rounding is monotone)
  if constexpr (RELU) v = __builtin_elementwise_max(v, half8{0, 0, 0, 0, 0, 0, 0, 0});
  b[s] = v;
}

// Layer l MFMAs of tile X; hand-off slot s of tile Y's layer LP (LP < 0: none)
// follows MFMA floor(s NM / NH).
template <class N, int l, int LP, bool RELU, bool BIAS, class WS>
__device__ __forceinline__ void stage_pair(const WS& ws, const half8 (&bX)[N::kMaxKC], f32x16 (&accX)[N::kMaxMT],
                                           const f32x16 (&accY)[N::kMaxMT], half8 (&bY)[N::kMaxKC]) {
  constexpr int NM = N::mt(l) * N::kc(l);
  constexpr int NH = LP >= 0 ? 2 * N::mt(LP < 0 ? 0 : LP) : 0;
  const f32x16 zero = {};
#pragma unroll
  for (int c = 0; c < N::kc(l); ++c) {
#pragma unroll
    for (int t = 0; t < N::mt(l); ++t) {
      const int i = c * N::mt(l) + t;
      const f32x16& cin = (BIAS || c > 0) ? accX[t] : zero;
      accX[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ws.get(N::frag_base(l) + t * N::kc(l) + c), bX[c], cin, 0, 0, 0);
      if constexpr (NH > 0) {
#pragma unroll
        for (int s = 0; s < NH; ++s)
          if ((s * NM) / NH == i) handoff_slot<N, LP < 0 ? 0 : LP, RELU>(s, accY, bY);
      }
    }
  }
}

// Layer 0 MFMAs of tile A, with tile B's input encoding right after the first.
template <class N, bool BIAS, class WS>
__device__ __forceinline__ void stage_pair_input(const WS& ws, const half8 (&bA)[N::kMaxKC], f32x16 (&accA)[N::kMaxMT],
                                                 const float (&pB)[N::kIn], int h, half8 (&bB)[N::kMaxKC]) {
  const f32x16 zero = {};
#pragma unroll
  for (int c = 0; c < N::kc(0); ++c) {
#pragma unroll
    for (int t = 0; t < N::mt(0); ++t) {
      const f32x16& cin = (BIAS || c > 0) ? accA[t] : zero;
      accA[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ws.get(N::frag_base(0) + t * N::kc(0) + c), bA[c], cin, 0, 0, 0);
      if (c == 0 && t == 0) build_input<N>(pB, h, bB);
    }
  }
}

// The whole chain for tiles A (input fragments in bA) and B (raw input pB).
// On return accA / accB hold the last layer's D of each tile.
template <class N, int l, bool RELU, bool BIAS, class WS>
__device__ __forceinline__ void run_pair(const WS& ws, const float (&pB)[N::kIn], int h, half8 (&bA)[N::kMaxKC],
                                         half8 (&bB)[N::kMaxKC], f32x16 (&accA)[N::kMaxMT],
                                         f32x16 (&accB)[N::kMaxMT], const float* sb) {
  if constexpr (BIAS) load_bias<N, l>(accA, sb, h);
  if constexpr (l == 0) stage_pair_input<N, BIAS>(ws, bA, accA, pB, h, bB);
  else stage_pair<N, l, l - 1, RELU, BIAS>(ws, bA, accA, accB, bB);
  if constexpr (BIAS) load_bias<N, l>(accB, sb, h);
  if constexpr (l + 1 < N::kL) {
    stage_pair<N, l, l, RELU, BIAS>(ws, bB, accB, accA, bA);
    run_pair<N, l + 1, RELU, BIAS>(ws, pB, h, bA, bB, accA, accB, sb);
  } else {
    stage_pair<N, l, -1, RELU, BIAS>(ws, bB, accB, accA, bA);
  }
}

// Output activation of the last layer (compile-time so that the unused heads
// cost nothing).  The transcendental heads use the hardware exp2/log2/rcp.
template <int ACT>
__device__ __forceinline__ float head_act(int channel, float v) {
  if constexpr (ACT == RDV_ACT_RELU) return fmaxf(v, 0.0f);
  else if constexpr (ACT == RDV_ACT_SOFTPLUS) return fast_softplus(v);
  else if constexpr (ACT == RDV_ACT_SIGMOID) return fast_sigmoid(v);
  else if constexpr (ACT == RDV_ACT_DENSITY_RGB) return channel == 0 ? fast_softplus(v) : fast_sigmoid(v);
  else return v;
}

// Stores the head values of one row (rows 32t + 8q + 4h + 0..3 of the last D).
template <class N>
__device__ __forceinline__ void store_head(float* __restrict__ yr, const f32x4 (&v)[N::mt(N::kL - 1)][4], int h) {
#pragma unroll
  for (int t = 0; t < N::mt(N::kL - 1); ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r0 = 32 * t + 8 * q + 4 * h;
      if (r0 < N::kOut) {
        if constexpr (N::kOut % 4 == 0) {
          // streaming (non-temporal) store: the output is not re-read by this kernel
          __builtin_nontemporal_store(v[t][q], reinterpret_cast<f32x4*>(yr + r0));
        } else {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj)
            if (r0 + jj < N::kOut) __builtin_nontemporal_store(v[t][q][jj], yr + r0 + jj);
        }
      }
    }
  }
}

// ----------------------------------------------------------------- kernel
// A zero the compiler cannot see through, re-materialised per loop iteration.
__device__ __forceinline__ int opaque_zero() {
  int z = 0;
  asm volatile("" : "+s"(z));
  return z;
}

}  // namespace rdv

#endif  // RDV_MLP_CORE_H
