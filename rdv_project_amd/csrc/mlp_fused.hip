// Fused fp16 matrix-core MLP: the whole layer chain evaluated per wave, weights
// resident in VGPRs for the life of the wave, activations passed from layer to
// layer in registers (the D -> B fragment identity of mlp_layout.h).
//
// Replaces the reference's LinearFast / ReLU megakernel
// (src/rdv/shaders/maps/linear_fast.h:39-100, relu.h:1-5, composite.h:8-12,
// map_evaluator.h:1-5), which staged a 16x16 weight tile through shared memory
// per (m0, n0, k0) with two barriers each, and re-quantised every layer input to
// fp16 (linear_fast.h:62).  The numerics here are the same: layer inputs and
// weights in fp16, products accumulated in fp32, fp32 bias, activation in fp32
// before the next rounding to fp16.
//
// Work decomposition: one 8-wave block per CU; each wave evaluates one 32-point
// tile (one MFMA N block) at a time, claiming tiles dynamically (see the kernel).
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

struct FusedArgs {
  const float* x;
  float* y;
  const uint8_t* packed;
  int64_t nrows;  // rows evaluated by this launch (starting at x / y)
  int act[RDV_MLP_MAX_LAYERS];
  MlpLayout lay;
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

// Where a wave's A fragments live: VGPRs for the life of the wave, or the
// block's LDS copy (fragment f is a conflict-free 1 KiB line, one
// ds_read_b128 per lane, read right before its MFMA).
template <class N>
struct RegWeights {
  half8 w[N::kFrags];
  __device__ __forceinline__ half8 get(int f) const { return w[f]; }
};
struct LdsWeights {
  const half8* sw;  // fragment f at sw[f * 64 + lane]
  int lane;
  __device__ __forceinline__ half8 get(int f) const { return sw[f * 64 + lane]; }
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

// Work decomposition.  One 512-thread block (8 waves, 2 per SIMD) per CU owns a
// contiguous range of 32-row tiles; its waves claim tiles one at a time from an
// LDS counter, so the two waves of a SIMD finish together (with a static split
// the SIMD arbiter's preference for older waves let one finish ~25% earlier,
// leaving the tail at one wave per SIMD).
//  - Weights: the block copies the packed A fragments into LDS once, and every
//    wave then reads its copy into VGPRs.  (2048 waves each pulling the same
//    26 KiB straight from L2 serialised on a few hot lines for ~3 us.)
//  - Input: at the top of an iteration a wave claims its next tile and issues
//    that tile's row loads into registers; at the bottom, a whole tile of work
//    later, it parks them in a wave-private LDS slot, which the next iteration
//    reads.  The wait for the load therefore lands where the data has long
//    arrived, and no barrier is needed after start-up.
//  - Output: each tile's store is issued after the next input has been parked,
//    so the wait that precedes the parking never covers a store younger than
//    a tile.
#ifndef RDV_MLP_WEIGHTS_IN_LDS
#define RDV_MLP_WEIGHTS_IN_LDS 1
#endif
// 4 waves per SIMD when the weights stay in LDS (<= 128 VGPRs), 2 when they
// are held in VGPRs.
constexpr int kWaves = RDV_MLP_WEIGHTS_IN_LDS ? 16 : 8;
constexpr int kThreads = 64 * kWaves;

template <class N, bool RELU, int HEAD_ACT>
__global__ __launch_bounds__(kThreads, 1) void mlp_fused_f16_kernel(FusedArgs a) {
  constexpr int D = N::kIn;
  constexpr int LL = N::kL - 1;
  constexpr int MTO = N::mt(LL);
  __shared__ float sb[N::kBias];
  __shared__ half8 sw[N::kFrags * 64];
  __shared__ float sx[kWaves][32 * D];  // each wave's parked input tile
  __shared__ int s_next;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h = lane >> 5, col = lane & 31;

  const int64_t ntiles = (a.nrows + 31) >> 5;
  const int64_t per_block = (ntiles + gridDim.x - 1) / gridDim.x;
  const int64_t t_begin = int64_t(blockIdx.x) * per_block;
  const int64_t t_end = t_begin + per_block < ntiles ? t_begin + per_block : ntiles;
  const int nt = int(t_end > t_begin ? t_end - t_begin : 0);  // this block's tiles
  // all biases zero (flag computed by the packer): skip seeding the accumulators
  const bool has_bias = (reinterpret_cast<const MlpPackHeader*>(a.packed)->flags & kMlpHasBias) != 0;

  // ---- start-up: biases and fragments -> LDS, counter reset
#pragma unroll
  for (int l = 0; l < N::kL; ++l) {
    const float* src = reinterpret_cast<const float*>(a.packed + a.lay.bias_off[l]);
    for (int i = threadIdx.x; i < 32 * N::mt(l); i += kThreads) sb[N::bias_base(l) + i] = src[i];
    const half8* fsrc = reinterpret_cast<const half8*>(a.packed + a.lay.frag_off[l]);
    for (int i = threadIdx.x; i < N::kc(l) * N::mt(l) * 64; i += kThreads) sw[N::frag_base(l) * 64 + i] = fsrc[i];
  }
  if (threadIdx.x == 0) s_next = 0;
  __syncthreads();

  auto claim = [&]() {
    int t = 0;
    if (lane == 0) t = atomicAdd(&s_next, 1);
    return __builtin_amdgcn_readfirstlane(t);
  };
  // Rows of block tile lt (clamped to valid rows: tiles past the end are never
  // computed, rows past the end of the last tile feed outputs that are not stored).
  const int64_t last = a.nrows - 1;
  auto load_tile = [&](int lt, float (&r)[D]) {
    int64_t row = (t_begin + (lt < nt ? lt : 0)) * 32 + col;
    row = row < last ? row : last;
#pragma unroll
    for (int d = 0; d < D; ++d) r[d] = __builtin_nontemporal_load(a.x + row * D + d);
  };
  auto park = [&](const float (&r)[D]) {
    if (h == 0) {
#pragma unroll
      for (int d = 0; d < D; ++d) sx[wave][col * D + d] = r[d];
    }
  };

  int cur = claim();
  {
    float r[D];
    load_tile(cur, r);
    park(r);
  }
#if !RDV_MLP_WEIGHTS_IN_LDS
  RegWeights<N> rw;
#pragma unroll
  for (int f = 0; f < N::kFrags; ++f) rw.w[f] = sw[f * 64 + lane];
#endif

  // Each tile's output is stored one iteration late, after the next park: the
  // wait preceding a park then never covers a store younger than a whole tile
  // (write acknowledgements under load take longer than one tile).
  f32x4 po[MTO][4];
  int64_t prow = -1;
  while (cur < nt) {
    const int nxt = claim();
    float r[D];
    load_tile(nxt, r);

    float p[D];
#pragma unroll
    for (int d = 0; d < D; ++d) p[d] = sx[wave][col * D + d];
    // The bias reads are loop-invariant; left visible, the compiler hoists all
    // of them out of the tile loop and pins 16 VGPRs per M tile.  A zero offset
    // laundered through an empty asm each iteration keeps them as per-tile LDS
    // reads straight into the accumulators.
    f32x16 accA[N::kMaxMT], accB[N::kMaxMT];
    half8 b[N::kMaxKC];
#if RDV_MLP_WEIGHTS_IN_LDS
    const LdsWeights ws{sw + opaque_zero(), lane};  // opaque offset keeps the reads in the loop
#else
    const RegWeights<N>& ws = rw;
#endif
    if (has_bias) {
      const float* sbt = sb + opaque_zero();
      load_bias<N, 0>(accA, sbt, h);
      build_input<N>(p, h, b);
      run_chain<N, 0, RELU, true>(ws, b, accA, accB, sbt, h);
    } else {
      build_input<N>(p, h, b);
      run_chain<N, 0, RELU, false>(ws, b, accA, accB, sb, h);
    }
    const f32x16 (&fin)[N::kMaxMT] = (LL % 2 == 0) ? accA : accB;
    f32x4 o[MTO][4];
#pragma unroll
    for (int t = 0; t < MTO; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          o[t][q][jj] = head_act<HEAD_ACT>(32 * t + 8 * q + 4 * h + jj, fin[t][4 * q + jj]);

    park(r);  // the next tile's input, loaded a whole tile ago
    if (prow >= 0 && prow < a.nrows) store_head<N>(a.y + prow * N::kOut, po, h);
#pragma unroll
    for (int t = 0; t < MTO; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) po[t][q] = o[t][q];
    prow = (t_begin + cur) * 32 + col;
    cur = nxt;
  }
  if (prow >= 0 && prow < a.nrows) store_head<N>(a.y + prow * N::kOut, po, h);
}

// ---------------------------------------------------------- instantiations
using NetRaw3_64x4_4 = Net<RDV_ENC_NONE, 3, 0, 4, 1, 2, 2, 2, 2, 1>;  // 3->64->64->64->64->4
using NetRaw3_64x3_4 = Net<RDV_ENC_NONE, 3, 0, 4, 1, 2, 2, 2, 1>;     // 3->64->64->64->4
using NetRaw3_64x2_4 = Net<RDV_ENC_NONE, 3, 0, 4, 1, 2, 2, 1>;        // 3->64->64->4
using NetRaw3_64x3_1 = Net<RDV_ENC_NONE, 3, 0, 1, 1, 2, 2, 2, 1>;     // 3->64->64->64->1
using NetFreq3x6_64x3_4 = Net<RDV_ENC_FREQ, 3, 6, 4, 3, 2, 2, 2, 1>;  // enc(39->48)->64->64->64->4
using NetFreq3x6_64x2_4 = Net<RDV_ENC_FREQ, 3, 6, 4, 3, 2, 2, 1>;     // enc(39->48)->64->64->4

typedef int (*FusedLauncher)(const FusedArgs&, int64_t nrows, hipStream_t);

template <class N, bool RELU, int HEAD_ACT>
int launch_fused(const FusedArgs& a, int64_t nrows, hipStream_t stream) {
  if (nrows <= 0) return RDV_OK;
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  const int64_t ntiles = (nrows + 31) / 32;
  // one 8-wave block per CU; never more waves than tiles
  int64_t blocks = di.cu_count;
  const int64_t need = (ntiles + kWaves - 1) / kWaves;
  if (need < blocks) blocks = need;
  mlp_fused_f16_kernel<N, RELU, HEAD_ACT><<<dim3(unsigned(blocks)), dim3(kThreads), 0, stream>>>(a);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

struct FusedEntry {
  int enc, in, oct, out, L, kc0, hidden_act, head_act;
  int mt[RDV_MLP_MAX_LAYERS];
  FusedLauncher fn;
  const char* name;
};

template <class N, bool RELU, int HEAD_ACT>
FusedEntry entry(const char* name) {
  FusedEntry e{};
  e.hidden_act = RELU ? RDV_ACT_RELU : RDV_ACT_NONE;
  e.head_act = HEAD_ACT;
  e.enc = N::kEnc;
  e.in = N::kIn;
  e.oct = N::kOct;
  e.out = N::kOut;
  e.L = N::kL;
  e.kc0 = N::kc(0);
  for (int i = 0; i < N::kL; ++i) e.mt[i] = N::mt(i);
  e.fn = &launch_fused<N, RELU, HEAD_ACT>;
  e.name = name;
  return e;
}

static const FusedEntry* fused_table(int* count) {
  static const FusedEntry table[] = {
      entry<NetRaw3_64x4_4, true, RDV_ACT_NONE>("mlp_fused_f16<raw3,64x4,4>"),
      entry<NetRaw3_64x3_4, true, RDV_ACT_NONE>("mlp_fused_f16<raw3,64x3,4>"),
      entry<NetRaw3_64x3_4, true, RDV_ACT_DENSITY_RGB>("mlp_fused_f16<raw3,64x3,4,density_rgb>"),
      entry<NetRaw3_64x2_4, true, RDV_ACT_NONE>("mlp_fused_f16<raw3,64x2,4>"),
      entry<NetRaw3_64x3_1, true, RDV_ACT_NONE>("mlp_fused_f16<raw3,64x3,1>"),
      entry<NetRaw3_64x3_1, true, RDV_ACT_SOFTPLUS>("mlp_fused_f16<raw3,64x3,1,softplus>"),
      entry<NetFreq3x6_64x3_4, true, RDV_ACT_NONE>("mlp_fused_f16<freq3x6,64x3,4>"),
      entry<NetFreq3x6_64x3_4, true, RDV_ACT_DENSITY_RGB>("mlp_fused_f16<freq3x6,64x3,4,density_rgb>"),
      entry<NetFreq3x6_64x2_4, true, RDV_ACT_NONE>("mlp_fused_f16<freq3x6,64x2,4>"),
  };
  *count = int(sizeof(table) / sizeof(table[0]));
  return table;
}

// Matrix-core instantiation serving `d`, or nullptr.
const FusedEntry* find_fused(const rdv_mlp_desc& d, const MlpLayout& lay) {
  for (int i = 0; i < d.n_layers; ++i)
    if (d.prec[i] != RDV_PREC_F16) return nullptr;
  int n = 0;
  const FusedEntry* t = fused_table(&n);
  for (int k = 0; k < n; ++k) {
    const FusedEntry& e = t[k];
    if (e.enc != d.encoding || e.in != d.in_features || e.L != d.n_layers) continue;
    if (e.enc == RDV_ENC_FREQ && e.oct != d.enc_octaves) continue;
    if (e.out != d.dims[d.n_layers] || e.kc0 != lay.kc[0] || e.head_act != d.act[d.n_layers - 1]) continue;
    bool ok = true;
    for (int i = 0; i < d.n_layers && ok; ++i) ok = e.mt[i] == lay.mt[i];
    for (int i = 0; i + 1 < d.n_layers && ok; ++i) ok = d.act[i] == e.hidden_act;
    if (ok) return &e;
  }
  return nullptr;
}

const char* fused_name(const FusedEntry* e) { return e ? e->name : nullptr; }

int launch_fused_entry(const FusedEntry* e, const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed,
                       const float* x, float* y, int64_t nrows, hipStream_t stream) {
  FusedArgs a;
  a.x = x;
  a.y = y;
  a.packed = static_cast<const uint8_t*>(packed);
  a.nrows = nrows;
  for (int i = 0; i < RDV_MLP_MAX_LAYERS; ++i) a.act[i] = i < d.n_layers ? d.act[i] : 0;
  a.lay = lay;
  return e->fn(a, nrows, stream);
}

}  // namespace rdv
