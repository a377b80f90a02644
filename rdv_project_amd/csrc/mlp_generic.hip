// Runtime-shaped fused fp16 MLP forward: every LinearFast chain without a
// compile-time instantiation (mlp_fused.hip) runs here on the matrix cores.
//
// Replaces, for those chains, the reference's LinearFast / ReLU megakernel
// (src/rdv/shaders/maps/linear_fast.h:39-100, which pads IN and OUT to 16 and
// runs coopMatMulAdd for any shape, linear_fast.h:29-30,61-98; relu.h,
// composite.h:8-12, map_evaluator.h:1-5).  Numerics are the LinearFast ones:
// fp16 layer inputs and weights, fp32 accumulation, fp32 bias, activation in
// fp32 before the next rounding to fp16.
//
// Work decomposition: one block per CU (persistent; 8 waves, or 4 for chains
// with a layer wider than 128), each block owns a
// contiguous range of 32-point tiles and its waves claim them from an LDS
// counter.  The chain's fragments and biases are staged into LDS once when
// they fit (dynamic LDS up to kGenLdsCap), else read from the packed block in
// global memory.  Layer 0's B fragments are built from the row in place: raw
// features (two 16-byte loads per K chunk when rows are 16-byte aligned) or
// the frequency encoding evaluated per slot.
#include "mlp_core.h"
#include "mlp_generic.h"

namespace rdv {

constexpr int64_t kGenLdsCap = 152 * 1024;

struct GenFwdArgs {
  const float* x;
  float* y;
  const uint8_t* packed;
  int64_t nrows;
  int vec_in;   // rows of x are 16-byte aligned and D % 4 == 0
  int vec_out;  // rows of y are 16-byte aligned and out % 4 == 0
  GenNet net;
};

template <int MT, bool LDSW>
__global__ __launch_bounds__(64 * gen_waves<MT>(), 1) void mlp_generic_f16_kernel(GenFwdArgs a) {
  constexpr int kGenWaves = gen_waves<MT>();
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ int s_next;
  const GenNet& g = a.net;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int h0 = lane >> 5, col = lane & 31;
  const bool has_bias = (reinterpret_cast<const MlpPackHeader*>(a.packed)->flags & kMlpHasBias) != 0;

  const half8* wsrc0;
  const float* bsrc0;
  if constexpr (LDSW) {
    gen_stage(a.packed, g, smem);
    wsrc0 = reinterpret_cast<const half8*>(smem);
    bsrc0 = reinterpret_cast<const float*>(smem + int64_t(g.n_frag) * 1024);
  } else {
    wsrc0 = reinterpret_cast<const half8*>(a.packed + g.frag_off0);
    bsrc0 = reinterpret_cast<const float*>(a.packed + g.bias_off0);
  }
  if (threadIdx.x == 0) s_next = kGenWaves;
  __syncthreads();

  const int64_t ntiles = (a.nrows + 31) >> 5;
  const int64_t per_block = (ntiles + gridDim.x - 1) / gridDim.x;
  const int64_t t_begin = int64_t(blockIdx.x) * per_block;
  const int64_t t_end = t_begin + per_block < ntiles ? t_begin + per_block : ntiles;
  const int nt = int(t_end > t_begin ? t_end - t_begin : 0);
  auto claim = [&]() {
    int t = 0;
    if (lane == 0) t = atomicAdd(&s_next, 1);
    return __builtin_amdgcn_readfirstlane(t);
  };
  const int D = g.D, OUT0 = g.out, LL = g.L - 1;

  for (int t = wave; t < nt; t = claim()) {
    // Values the compiler cannot see through, re-made per tile: without them it
    // hoists every lane mask and address of the head stores and bias reads out
    // of the loop, and spills them.
    const int z = opaque_zero();
    int h = h0;
    asm volatile("" : "+v"(h));
    const half8* wsrc = wsrc0 + z;
    const float* bsrc = bsrc0 + z;
    const int OUT = OUT0 + z;
    auto wf = [&](int f) { return wsrc[f * 64 + lane]; };
    const int64_t row = (t_begin + t) * 32 + col;
    const int64_t rc = row < a.nrows ? row : a.nrows - 1;  // clamped: every load in bounds
    const float* xr = a.x + rc * D;
    auto get = [&](int d) { return xr[d]; };
    auto l0 = [&](int c) -> half8 {
      if (g.enc == RDV_ENC_NONE && a.vec_in) {
        const int f = 16 * c + 8 * h;
        const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
        const f32x4 v0 = f < D ? *reinterpret_cast<const f32x4*>(xr + f) : zero4;
        const f32x4 v1 = f + 4 < D ? *reinterpret_cast<const f32x4*>(xr + f + 4) : zero4;
        half8 b;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          b[j] = half_t(v0[j]);
          b[4 + j] = half_t(v1[j]);
        }
        return b;
      }
      return gen_l0_chunk(g, c, h, get);
    };
    const GenCtx cx{bsrc, has_bias, h};
    auto sink = [&](const auto& acc) {
      constexpr int M = sizeof(acc) / sizeof(acc[0]);
      // the output masks and addresses are formed here, after the chain's
      // memory reads, not hoisted above the chain where they would stay live
      int hs = h;
      asm volatile("" : "+v"(hs) : : "memory");
      if (row < a.nrows) {
        float* yr = a.y + row * OUT;
        const int act = g.act[LL];
#pragma unroll
        for (int tt = 0; tt < M; ++tt) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int r0 = 32 * tt + 8 * q + 4 * hs;
            if (r0 < OUT) {
              f32x4 v;
#pragma unroll
              for (int jj = 0; jj < 4; ++jj) v[jj] = gen_head_act(act, r0 + jj, acc[tt][4 * q + jj]);
              if (a.vec_out) {
                __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(yr + r0));
              } else {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                  if (r0 + jj < OUT) yr[r0 + jj] = v[jj];
              }
            }
          }
        }
      }
    };
    gen_chain<MT>(g, cx, wf, l0, sink);
  }
}

template <int MT, bool LDSW>
static int launch_generic_t(const GenFwdArgs& a, int64_t blocks, size_t lds, hipStream_t stream) {
  static bool attr = false;
  if (LDSW && !attr) {
    RDV_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&mlp_generic_f16_kernel<MT, LDSW>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(kGenLdsCap)));
    attr = true;
  }
  mlp_generic_f16_kernel<MT, LDSW><<<dim3(unsigned(blocks)), dim3(64 * gen_waves<MT>()), lds, stream>>>(a);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

// True when the generic matrix-core kernel serves `d` (every layer LinearFast).
bool generic_f16_supported(const rdv_mlp_desc& d) {
  for (int i = 0; i < d.n_layers; ++i)
    if (d.prec[i] != RDV_PREC_F16) return false;
  return true;
}

const char* generic_f16_name(const rdv_mlp_desc& d, const MlpLayout& lay) {
  GenNet g;
  gen_net(d, lay, &g);
  const bool lds = gen_lds_bytes(g) <= kGenLdsCap;
  static const char* names[2][4] = {
      {"mlp_generic_f16<1,global>", "mlp_generic_f16<2,global>", "mlp_generic_f16<4,global>",
       "mlp_generic_f16<8,global>"},
      {"mlp_generic_f16<1,lds>", "mlp_generic_f16<2,lds>", "mlp_generic_f16<4,lds>", "mlp_generic_f16<8,lds>"}};
  const int m = gen_mt_bound(g);
  return names[lds ? 1 : 0][m == 1 ? 0 : m == 2 ? 1 : m == 4 ? 2 : 3];
}

int launch_mlp_generic_f16(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, const float* x, float* y,
                           int64_t nrows, hipStream_t stream) {
  if (nrows <= 0) return RDV_OK;
  DeviceInfo di;
  int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  GenFwdArgs a;
  a.x = x;
  a.y = y;
  a.packed = static_cast<const uint8_t*>(packed);
  a.nrows = nrows;
  gen_net(d, lay, &a.net);
  a.vec_in = (d.encoding == RDV_ENC_NONE && d.in_features % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0) ? 1 : 0;
  a.vec_out = (a.net.out % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0) ? 1 : 0;
  const int64_t ntiles = (nrows + 31) / 32;
  const int mtb = gen_mt_bound(a.net);
  const int waves = mtb >= 8 ? gen_waves<8>() : gen_waves<1>();
  int64_t blocks = di.cu_count;
  const int64_t need = (ntiles + waves - 1) / waves;
  if (need < blocks) blocks = need;
  const int64_t lds = gen_lds_bytes(a.net);
  const bool use_lds = lds <= kGenLdsCap;
  switch (mtb) {
    case 1: return use_lds ? launch_generic_t<1, true>(a, blocks, size_t(lds), stream)
                           : launch_generic_t<1, false>(a, blocks, 0, stream);
    case 2: return use_lds ? launch_generic_t<2, true>(a, blocks, size_t(lds), stream)
                           : launch_generic_t<2, false>(a, blocks, 0, stream);
    case 4: return use_lds ? launch_generic_t<4, true>(a, blocks, size_t(lds), stream)
                           : launch_generic_t<4, false>(a, blocks, 0, stream);
    default: return use_lds ? launch_generic_t<8, true>(a, blocks, size_t(lds), stream)
                            : launch_generic_t<8, false>(a, blocks, 0, stream);
  }
}

}  // namespace rdv
