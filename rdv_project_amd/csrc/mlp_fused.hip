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
// Work decomposition: each wave owns a 32-point tile at a time (one MFMA N
// block) and walks tiles with a grid stride; the grid is sized to the resident
// wave count so every wave loads its weights exactly once.
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
          // sin(2^k pi p) = sin(2 pi * 2^(k-1) p); v_sin/v_cos take revolutions,
          // and the power-of-two scale is exact.
          const float s0 = __builtin_ldexpf(1.0f, i - 1);
          const float s1 = __builtin_ldexpf(1.0f, H0 + i - 1);
          const float arg = (h ? s1 : s0) * p[d];
          v = is_cos ? __builtin_amdgcn_cosf(arg) : __builtin_amdgcn_sinf(arg);
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
template <class N, int l>
__device__ __forceinline__ void run_layer(const half8 (&w)[N::kFrags], const half8 (&b)[N::kMaxKC],
                                          f32x16 (&acc)[N::kMaxMT], const float* sb, int h) {
  // accumulators start at the bias (rows 32t + 8q + 4h + 0..3 are contiguous)
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
#pragma unroll
  for (int c = 0; c < N::kc(l); ++c) {
#pragma unroll
    for (int t = 0; t < N::mt(l); ++t) {
      acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[N::frag_base(l) + t * N::kc(l) + c], b[c], acc[t], 0, 0, 0);
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

template <class N, int l, bool RELU>
__device__ __forceinline__ void run_chain(const half8 (&w)[N::kFrags], half8 (&b)[N::kMaxKC],
                                          f32x16 (&acc)[N::kMaxMT], const float* sb, int h) {
  run_layer<N, l>(w, b, acc, sb, h);
  if constexpr (l + 1 < N::kL) {
    to_next<N, l, RELU>(acc, b);
    run_chain<N, l + 1, RELU>(w, b, acc, sb, h);
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

// ----------------------------------------------------------------- kernel
template <class N, bool RELU, int HEAD_ACT>
__global__ __launch_bounds__(256, 2) void mlp_fused_f16_kernel(FusedArgs a) {
  constexpr int D = N::kIn;
  constexpr int LL = N::kL - 1;
  __shared__ float sb[N::kBias];
  const int lane = threadIdx.x & 63;
  const int h = lane >> 5, col = lane & 31;

  // padded biases -> LDS
#pragma unroll
  for (int l = 0; l < N::kL; ++l) {
    const float* src = reinterpret_cast<const float*>(a.packed + a.lay.bias_off[l]);
    for (int i = threadIdx.x; i < 32 * N::mt(l); i += blockDim.x) sb[N::bias_base(l) + i] = src[i];
  }
  // A fragments -> registers, once per wave
  half8 w[N::kFrags];
#pragma unroll
  for (int l = 0; l < N::kL; ++l) {
    const half8* src = reinterpret_cast<const half8*>(a.packed + a.lay.frag_off[l]);
#pragma unroll
    for (int f = 0; f < N::kc(l) * N::mt(l); ++f) w[N::frag_base(l) + f] = src[f * 64 + lane];
  }
  __syncthreads();

  const int64_t ntiles = (a.nrows + 31) >> 5;
  const int64_t nwaves = (int64_t(gridDim.x) * blockDim.x) >> 6;
  int64_t tile = (int64_t(blockIdx.x) * blockDim.x + threadIdx.x) >> 6;

  float p[D];
  {
    const int64_t row = tile * 32 + col;
    const bool ok = tile < ntiles && row < a.nrows;
#pragma unroll
    for (int d = 0; d < D; ++d) p[d] = ok ? a.x[row * D + d] : 0.0f;
  }
  for (; tile < ntiles; tile += nwaves) {
    float pc[D];
#pragma unroll
    for (int d = 0; d < D; ++d) pc[d] = p[d];
    {  // prefetch the next tile's input
      const int64_t row = (tile + nwaves) * 32 + col;
      const bool ok = row < a.nrows;
#pragma unroll
      for (int d = 0; d < D; ++d) p[d] = ok ? a.x[row * D + d] : 0.0f;
    }
    half8 b[N::kMaxKC];
    build_input<N>(pc, h, b);
    f32x16 acc[N::kMaxMT];
    // The bias reads are loop-invariant; left visible, the compiler hoists all
    // of them out of the tile loop and pins 16 VGPRs per M tile.  An opaque zero
    // offset keeps them as per-tile LDS reads straight into the accumulators.
    int sb_off = 0;
    asm volatile("" : "+s"(sb_off));
    run_chain<N, 0, RELU>(w, b, acc, sb + sb_off, h);

    // head: rows 32t + 8q + 4h + 0..3 of point `row`
    const int64_t row = tile * 32 + col;
    if (row < a.nrows) {
      float* yr = a.y + row * N::kOut;
#pragma unroll
      for (int t = 0; t < N::mt(LL); ++t) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r0 = 32 * t + 8 * q + 4 * h;
          if (r0 < N::kOut) {
            f32x4 v;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) v[jj] = head_act<HEAD_ACT>(r0 + jj, acc[t][4 * q + jj]);
            if constexpr (N::kOut % 4 == 0) {
              *reinterpret_cast<f32x4*>(yr + r0) = v;
            } else {
#pragma unroll
              for (int jj = 0; jj < 4; ++jj)
                if (r0 + jj < N::kOut) yr[r0 + jj] = v[jj];
            }
          }
        }
      }
    }
  }
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
  // 2 resident 256-thread blocks per CU (launch bounds); never more waves than tiles
  int64_t blocks = int64_t(2) * di.cu_count;
  const int64_t need = (ntiles + 3) / 4;
  if (need < blocks) blocks = need;
  mlp_fused_f16_kernel<N, RELU, HEAD_ACT><<<dim3(unsigned(blocks)), dim3(256), 0, stream>>>(a);
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
